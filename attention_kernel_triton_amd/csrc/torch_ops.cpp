// Compiled host layer of the hot entry points (prefill, dense / paged /
// sparse / MagicPIG decode, kept-index selection): the same checks, output allocation, stream and
// workspace handling as the package's Python wrappers, done in C++ so a
// drop-in call costs the host a few microseconds.  It calls the C ABI of
// libakt_amd.so (include/akt_amd.h) and nothing else; there is no fallback.
//
// Errors keep the Python wrappers' types: TypeError for dtypes, ValueError
// for devices and shapes, RuntimeError (with akt_last_error()) when the
// library rejects a call.  The reference's own shape asserts stay in the
// drop-in modules.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/extension.h>

#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/akt_amd.h"

namespace py = pybind11;

namespace {

const char* rc_name(int rc) {
  switch (rc) {
    case AKT_ERR_INVALID_ARGUMENT: return "invalid argument";
    case AKT_ERR_UNSUPPORTED: return "unsupported";
    case AKT_ERR_WORKSPACE: return "workspace";
    case AKT_ERR_HIP: return "HIP error";
  }
  return "error";
}

void check_rc(int rc, const char* what) {
  if (rc != AKT_OK)
    throw std::runtime_error(std::string(what) + " failed (" + rc_name(rc) + "): " +
                             akt_last_error());
}

std::string dev_str(const at::Tensor& t) { return t.device().str(); }

void need_gpu(const char* name, const at::Tensor& t) {
  if (!t.is_cuda())
    throw py::value_error(std::string(name) + " must be on a ROCm GPU device, got " + dev_str(t));
}

void same_device(const char* name, const at::Tensor& t, const at::Device& dev) {
  if (t.device() != dev)
    throw py::value_error(std::string(name) + " is on " + dev_str(t) + ", expected " + dev.str());
}

// Tensor of 2-byte elements with unit innermost stride and 16-byte aligned
// rows (a contiguous copy otherwise).
at::Tensor rows16(const at::Tensor& t) {
  bool ok = t.dim() >= 1 && t.stride(-1) == 1 &&
            (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) == 0;
  for (int64_t i = 0; ok && i + 1 < t.dim(); ++i) ok = (t.stride(i) * 2) % 16 == 0;
  return ok ? t : t.contiguous();
}

// fp16 tensor, as rows16.
at::Tensor half_rows(const char* name, const at::Tensor& t) {
  need_gpu(name, t);
  if (t.scalar_type() != at::kHalf)
    throw py::type_error(std::string(name) + " must be float16, got " +
                         std::string(c10::toString(t.scalar_type())));
  return rows16(t);
}

// fp16 or bf16 tensor of the given type, as rows16.
at::Tensor half_or_bf16_rows(const char* name, const at::Tensor& t, at::ScalarType want) {
  need_gpu(name, t);
  if (t.scalar_type() != want)
    throw py::type_error(std::string(name) + " must be " + std::string(c10::toString(want)) +
                         " like Q, got " + std::string(c10::toString(t.scalar_type())));
  return rows16(t);
}

at::Tensor int32_on(const char* name, const at::Tensor& t, const at::Device& dev) {
  need_gpu(name, t);
  same_device(name, t, dev);
  if (t.scalar_type() != at::kInt)
    throw py::type_error(std::string(name) + " must be int32, got " +
                         std::string(c10::toString(t.scalar_type())));
  return t;
}

void* ptr(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// Shape agreement of a dense Q / K / V triple, checked before devices and
// types (so a mismatch is reported as one on any device): 4-D tensors, K and
// V of one shape [B, Hkv, S, D] with Q's batch and head dim, and, for
// prefill, Q's sequence length.  The kernels size every K and V read from Q's
// and K's shapes, so a shorter V would otherwise be read past its end.
void check_dense_shapes(const at::Tensor& Q, const at::Tensor& K, const at::Tensor& V,
                        bool same_seq) {
  if (Q.dim() != 4 || K.dim() != 4 || V.dim() != 4)
    throw py::value_error("Q, K and V must be 4-D");
  if (K.sizes() != V.sizes())
    throw py::value_error("K and V must have one shape, got K " + c10::str(K.sizes()) + " and V " +
                          c10::str(V.sizes()));
  if (K.size(0) != Q.size(0) || K.size(3) != Q.size(3) || (same_seq && K.size(2) != Q.size(2)))
    throw py::value_error("K " + c10::str(K.sizes()) + " does not match Q " +
                          c10::str(Q.sizes()) +
                          (same_seq ? " in batch, sequence length or head dim"
                                    : " in batch or head dim"));
}

struct Strides {
  int64_t v[5] = {0, 0, 0, 0, 0};
};
Strides strides_of(const at::Tensor& t) {
  Strides s;
  for (int64_t i = 0; i < t.dim() && i < 5; ++i) s.v[i] = t.stride(i);
  return s;
}

// PyTorch on ROCm reports HIP devices as device type "cuda"; its HIP stream
// and device-guard types that accept them are the *MasqueradingAsCUDA ones.
hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

// One zero-initialised split-KV workspace per (device, stream), grown by
// doubling: the C ABI needs the counter header zero before first use (every
// call leaves it zero) and a workspace used only by calls ordered on one
// stream.
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, at::Tensor> g_ws;

at::Tensor workspace(size_t nbytes, const at::Device& dev, hipStream_t st) {
  if (nbytes == 0) return at::Tensor();
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto key = std::make_pair((int)dev.index(), st);
  auto it = g_ws.find(key);
  if (it != g_ws.end() && (size_t)it->second.numel() >= nbytes) return it->second;
  const int64_t old = it == g_ws.end() ? 0 : it->second.numel();
  const int64_t size = std::max<int64_t>((int64_t)nbytes, 2 * old);
  at::Tensor buf = at::zeros({size}, at::TensorOptions().dtype(at::kByte).device(dev));
  g_ws[key] = buf;
  return buf;
}

py::object result(const at::Tensor& o, const at::Tensor& lse, bool return_lse) {
  if (return_lse) return py::make_tuple(o, lse);
  return py::cast(o);
}

// --------------------------------------------------------------------------- prefill
py::object prefill(const at::Tensor& Q_, const at::Tensor& K_, const at::Tensor& V_, bool causal,
                   double softmax_scale, const c10::optional<at::Tensor>& varlen_,
                   bool return_lse) {
  check_dense_shapes(Q_, K_, V_, true);
  need_gpu("Q", Q_);
  const at::ScalarType dt = Q_.scalar_type();
  if (dt != at::kHalf && dt != at::kBFloat16)
    throw py::type_error("Q must be float16 or bfloat16, got " + std::string(c10::toString(dt)));
  at::Tensor Q = rows16(Q_), K = half_or_bf16_rows("K", K_, dt), V = half_or_bf16_rows("V", V_, dt);
  const at::Device dev = Q.device();
  same_device("K", K, dev);
  same_device("V", V, dev);
  const int dtype = dt == at::kBFloat16 ? AKT_DTYPE_BF16 : AKT_DTYPE_F16;
  const int64_t B = Q.size(0), H = Q.size(1), S = Q.size(2), D = Q.size(3);
  const DeviceGuard guard(dev);
  at::Tensor O = at::empty({B, H, S, D}, Q.options());
  const void* vptr = nullptr;
  int vbits = 0;
  at::Tensor varlen;
  if (varlen_.has_value() && varlen_->defined()) {
    varlen = *varlen_;
    need_gpu("varlen", varlen);
    if (varlen.scalar_type() != at::kInt && varlen.scalar_type() != at::kLong)
      throw py::type_error("varlen must be int32 or int64, got " +
                           std::string(c10::toString(varlen.scalar_type())));
    if (varlen.numel() != B)
      throw py::value_error("varlen must have " + std::to_string(B) + " entries, got " +
                            std::to_string(varlen.numel()));
    varlen = varlen.contiguous();
    vptr = varlen.data_ptr();
    vbits = varlen.scalar_type() == at::kLong ? 64 : 32;
  }
  const Strides qs = strides_of(Q), ks = strides_of(K), vs = strides_of(V), os = strides_of(O);
  hipStream_t st = stream_of(Q);
  at::Tensor lse;
  Strides ls;
  if (return_lse) {
    lse = at::empty({B, H, S}, Q.options().dtype(at::kFloat));
    ls = strides_of(lse);
  }
  check_rc(akt_prefill_fwd_ex(ptr(Q), ptr(K), ptr(V), ptr(O), (float*)ptr(lse), B, H, K.size(1),
                              S, D, qs.v, ks.v, vs.v, os.v, return_lse ? ls.v : nullptr,
                              (float)softmax_scale, causal ? 1 : 0, vptr, vbits, dtype, st),
           "akt_prefill_fwd_ex");
  return result(O, lse, return_lse);
}

// --------------------------------------------------------------------------- dense decode
py::object decode(const at::Tensor& q_, const at::Tensor& K_, const at::Tensor& V_,
                  double softmax_scale, bool return_lse, int64_t chunk_tokens) {
  check_dense_shapes(q_, K_, V_, false);
  at::Tensor q = half_rows("q", q_), K = half_rows("K", K_), V = half_rows("V", V_);
  const at::Device dev = q.device();
  same_device("K", K, dev);
  same_device("V", V, dev);
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(3), Hkv = K.size(1), S = K.size(2);
  const DeviceGuard guard(dev);
  at::Tensor o = at::empty({B, Hq, 1, D}, q.options());
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq}, q.options().dtype(at::kFloat));
  hipStream_t st = stream_of(q);
  const size_t ws_n = akt_decode_workspace_size(B, Hq, Hkv, S, D, chunk_tokens);
  at::Tensor ws = workspace(ws_n, dev, st);
  const Strides qs = strides_of(q), ks = strides_of(K), vs = strides_of(V);
  check_rc(akt_decode_fwd(ptr(q), ptr(K), ptr(V), ptr(o), (float*)ptr(lse), B, Hq, Hkv, S, D,
                          qs.v, ks.v, vs.v, (float)softmax_scale, chunk_tokens, ptr(ws), ws_n, st),
           "akt_decode_fwd");
  return result(o, lse, return_lse);
}

// --------------------------------------------------------------------------- paged decode
py::object decode_paged(const at::Tensor& q_, const at::Tensor& pool_, const at::Tensor& indptr_,
                        const at::Tensor& indices_, const at::Tensor& last_,
                        const c10::optional<double>& softmax_scale, bool return_lse,
                        int64_t chunk_tokens) {
  at::Tensor q = half_rows("q", q_), pool = half_rows("paged_kv_cache", pool_);
  const at::Device dev = q.device();
  same_device("paged_kv_cache", pool, dev);
  at::Tensor indptr = int32_on("kv_page_indptr", indptr_, dev).contiguous();
  at::Tensor indices = int32_on("kv_page_indices", indices_, dev).contiguous();
  at::Tensor last = int32_on("kv_last_page_len", last_, dev).contiguous();
  if (q.dim() != 3 && q.dim() != 4) throw py::value_error("q must be [B, Hq, (1,) D]");
  if (pool.dim() != 5) throw py::value_error("paged_kv_cache must be [P, 2, Hkv, page, D]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(-1);
  at::Tensor q4 = q.dim() == 4 ? q : q.unsqueeze(2);
  const int64_t P = pool.size(0), Hkv = pool.size(2), page = pool.size(3);
  if (pool.size(4) != D)
    throw py::value_error("head_dim mismatch: q has " + std::to_string(D) + ", cache has " +
                          std::to_string(pool.size(4)));
  if (indptr.numel() != B + 1 || last.numel() != B)
    throw py::value_error("kv_page_indptr must have B+1 and kv_last_page_len B entries");
  const float scale = softmax_scale.has_value() ? (float)*softmax_scale
                                                : (float)(1.0 / std::sqrt((double)D));
  const DeviceGuard guard(dev);
  at::Tensor o = at::empty({B, Hq, D}, q.options());
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq}, q.options().dtype(at::kFloat));
  const int64_t total = indices.numel();
  hipStream_t st = stream_of(q);
  const size_t ws_n = akt_decode_paged_workspace_size(B, Hq, Hkv, D, page, total, chunk_tokens);
  at::Tensor ws = workspace(ws_n, dev, st);
  const Strides qs = strides_of(q4), ps = strides_of(pool);
  check_rc(akt_decode_paged_fwd(ptr(q4), ptr(pool), (const int32_t*)ptr(indptr),
                                (const int32_t*)ptr(indices), (const int32_t*)ptr(last), ptr(o),
                                (float*)ptr(lse), B, Hq, Hkv, D, page, total, P, qs.v, ps.v, scale,
                                chunk_tokens, ptr(ws), ws_n, st),
           "akt_decode_paged_fwd");
  return result(o, lse, return_lse);
}

// --------------------------------------------------------------------------- sparse decodes
struct SparseMeta {
  at::Tensor ind, nnz;
  int64_t ist[2], nst[2];
};

SparseMeta sparse_meta(const at::Tensor& sparse_ind, const at::Tensor& sparse_nnz,
                       const at::Device& dev, int64_t B, int64_t Hq) {
  SparseMeta m;
  m.ind = int32_on("sparse_ind", sparse_ind, dev);
  m.nnz = int32_on("sparse_nnz", sparse_nnz, dev);
  if (m.ind.dim() != 3 || m.ind.size(0) != B || m.ind.size(1) != Hq)
    throw py::value_error("sparse_ind must be [B=" + std::to_string(B) + ", H=" +
                          std::to_string(Hq) + ", L_max]");
  if (m.ind.stride(2) != 1) m.ind = m.ind.contiguous();
  if (m.nnz.dim() < 2 || m.nnz.size(0) != B || m.nnz.size(1) != Hq ||
      (m.nnz.dim() == 3 && m.nnz.size(2) != 1))
    throw py::value_error("sparse_nnz must be [B=" + std::to_string(B) + ", H=" +
                          std::to_string(Hq) + "(, 1)]");
  m.ist[0] = m.ind.stride(0);
  m.ist[1] = m.ind.stride(1);
  m.nst[0] = m.nnz.stride(0);
  m.nst[1] = m.nnz.stride(1);
  return m;
}

py::object sparse_decode(const at::Tensor& q_, const at::Tensor& K_, const at::Tensor& V_,
                         const at::Tensor& sparse_ind, const at::Tensor& sparse_nnz,
                         double softmax_scale, bool return_lse, int64_t num_splits) {
  check_dense_shapes(q_, K_, V_, false);
  at::Tensor q = half_rows("q", q_), K = half_rows("K", K_), V = half_rows("V", V_);
  const at::Device dev = q.device();
  same_device("K", K, dev);
  same_device("V", V, dev);
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(3), Hkv = K.size(1), S = K.size(2);
  SparseMeta m = sparse_meta(sparse_ind, sparse_nnz, dev, B, Hq);
  const int64_t L = m.ind.size(2);
  const DeviceGuard guard(dev);
  at::Tensor o = at::empty({B, Hq, 1, D}, q.options());
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq}, q.options().dtype(at::kFloat));
  hipStream_t st = stream_of(q);
  const size_t ws_n = akt_sparse_decode_workspace_size(B, Hq, D, L, num_splits);
  at::Tensor ws = workspace(ws_n, dev, st);
  const Strides qs = strides_of(q), ks = strides_of(K), vs = strides_of(V);
  check_rc(akt_sparse_decode_fwd(ptr(q), ptr(K), ptr(V), (const int32_t*)ptr(m.ind),
                                 (const int32_t*)ptr(m.nnz), ptr(o), (float*)ptr(lse), B, Hq, Hkv,
                                 S, D, L, qs.v, ks.v, vs.v, m.ist, m.nst, (float)softmax_scale,
                                 num_splits, ptr(ws), ws_n, st),
           "akt_sparse_decode_fwd");
  return result(o, lse, return_lse);
}

py::object sparse_decode_paged(const at::Tensor& q_, const at::Tensor& pool_,
                               const at::Tensor& indptr_, const at::Tensor& indices_,
                               const at::Tensor& sparse_ind, const at::Tensor& sparse_nnz,
                               const c10::optional<double>& softmax_scale, bool return_lse,
                               int64_t num_splits, const c10::optional<at::Tensor>& lsh_k,
                               const c10::optional<at::Tensor>& lsh_l) {
  at::Tensor q = half_rows("q", q_), pool = half_rows("paged_kv_cache", pool_);
  const at::Device dev = q.device();
  same_device("paged_kv_cache", pool, dev);
  at::Tensor indptr = int32_on("kv_page_indptr", indptr_, dev).contiguous();
  at::Tensor indices = int32_on("kv_page_indices", indices_, dev).contiguous();
  if (q.dim() != 3 && q.dim() != 4) throw py::value_error("q must be [B, Hq, (1,) D]");
  if (pool.dim() != 5) throw py::value_error("paged_kv_cache must be [P, 2, Hkv, page, D]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(-1);
  at::Tensor q4 = q.dim() == 4 ? q : q.unsqueeze(2);
  const int64_t P = pool.size(0), Hkv = pool.size(2), page = pool.size(3);
  if (pool.size(4) != D)
    throw py::value_error("head_dim mismatch: q has " + std::to_string(D) + ", cache has " +
                          std::to_string(pool.size(4)));
  if (indptr.numel() != B + 1) throw py::value_error("kv_page_indptr must have B+1 entries");
  SparseMeta m = sparse_meta(sparse_ind, sparse_nnz, dev, B, Hq);
  const int64_t L = m.ind.size(2);
  const bool magic = lsh_k.has_value() && lsh_k->defined();
  at::Tensor lk, ll;
  if (magic) {
    if (!lsh_l.has_value() || !lsh_l->defined()) throw py::value_error("MagicPIG L is required");
    const std::pair<const char*, const at::Tensor*> kl[2] = {{"K", &*lsh_k}, {"L", &*lsh_l}};
    for (const auto& e : kl) {
      need_gpu(e.first, *e.second);
      if (e.second->scalar_type() != at::kFloat || e.second->dim() != 2 ||
          e.second->size(0) != B || e.second->size(1) != Hq)
        throw py::value_error(std::string("MagicPIG ") + e.first + " must be float32 [" +
                              std::to_string(B) + ", " + std::to_string(Hq) + "]");
    }
    lk = lsh_k->contiguous();
    ll = lsh_l->contiguous();
  }
  const DeviceGuard guard(dev);
  at::Tensor o = at::empty({B, Hq, D}, q.options());
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq}, q.options().dtype(at::kFloat));
  hipStream_t st = stream_of(q);
  const size_t ws_n = akt_sparse_decode_workspace_size(B, Hq, D, L, num_splits);
  at::Tensor ws = workspace(ws_n, dev, st);
  const Strides qs = strides_of(q4), ps = strides_of(pool);
  if (!magic) {
    const float scale = softmax_scale.has_value() ? (float)*softmax_scale
                                                  : (float)(1.0 / std::sqrt((double)D));
    check_rc(akt_sparse_decode_paged_fwd(ptr(q4), ptr(pool), (const int32_t*)ptr(indptr),
                                         (const int32_t*)ptr(indices), (const int32_t*)ptr(m.ind),
                                         (const int32_t*)ptr(m.nnz), ptr(o), (float*)ptr(lse), B,
                                         Hq, Hkv, D, page, P, L, qs.v, ps.v, m.ist, m.nst, scale,
                                         num_splits, ptr(ws), ws_n, st),
             "akt_sparse_decode_paged_fwd");
  } else {
    check_rc(akt_magicpig_decode_paged_fwd(ptr(q4), ptr(pool), (const int32_t*)ptr(indptr),
                                           (const int32_t*)ptr(indices),
                                           (const int32_t*)ptr(m.ind), (const int32_t*)ptr(m.nnz),
                                           (const float*)ptr(lk), (const float*)ptr(ll), ptr(o),
                                           (float*)ptr(lse), B, Hq, Hkv, D, page, P, L, qs.v, ps.v,
                                           m.ist, m.nst, num_splits, ptr(ws), ws_n, st),
             "akt_magicpig_decode_paged_fwd");
  }
  return result(o, lse, return_lse);
}

// --------------------------------------------------------------------------- kept indices
// Sorted kept-token index lists from a keep mask or uniform draws (the checks
// and outputs of _ops.kept_indices, in C++ so a call costs the host a few
// microseconds and back-to-back selections keep the GPU busy).
py::tuple kept_indices(int64_t l_max, const c10::optional<at::Tensor>& mask_,
                       const c10::optional<at::Tensor>& uniform_,
                       const c10::optional<double>& kept_ratio,
                       const c10::optional<at::Tensor>& row_len_, bool ensure_nonempty) {
  const bool has_mask = mask_.has_value() && mask_->defined();
  const bool has_uni = uniform_.has_value() && uniform_->defined();
  if (has_mask == has_uni) throw py::value_error("pass exactly one of mask= or uniform=");
  if (l_max < 0) throw py::value_error("l_max must be >= 0");
  const at::Tensor& src = has_mask ? *mask_ : *uniform_;
  need_gpu(has_mask ? "mask" : "uniform", src);
  if (src.dim() < 1) throw py::value_error("the keep source must have a last (token) dimension");
  const at::Device dev = src.device();
  std::vector<int64_t> lead(src.sizes().begin(), src.sizes().end() - 1);
  const int64_t n = src.size(-1);
  int64_t rows = 1;
  for (int64_t x : lead) rows *= x;
  at::Tensor rl;
  if (row_len_.has_value() && row_len_->defined()) {
    rl = int32_on("row_len", *row_len_, dev).contiguous();
    if (rl.numel() != rows) throw py::value_error("row_len must have one entry per row");
  }
  const DeviceGuard guard(dev);
  std::vector<int64_t> ishape = lead, nshape = lead;
  ishape.push_back(l_max);
  nshape.push_back(1);
  at::Tensor ind = at::empty(ishape, src.options().dtype(at::kInt));
  at::Tensor nnz = at::empty(nshape, src.options().dtype(at::kInt));
  hipStream_t st = stream_of(src);
  if (has_mask) {
    at::Tensor m = src.reshape({rows, n});
    if (m.scalar_type() == at::kBool) m = m.view(at::kByte);
    if (m.scalar_type() != at::kByte) throw py::type_error("mask must be bool or uint8");
    m = m.contiguous();
    check_rc(akt_kept_index_from_mask((const uint8_t*)ptr(m), rows, n, n,
                                      (const int32_t*)ptr(rl), (int32_t*)ptr(ind), l_max,
                                      (int32_t*)ptr(nnz), ensure_nonempty ? 1 : 0, st),
             "akt_kept_index_from_mask");
  } else {
    if (!kept_ratio.has_value()) throw py::value_error("kept_ratio is required with uniform=");
    at::Tensor u = src.reshape({rows, n});
    if (u.scalar_type() != at::kFloat) throw py::type_error("uniform must be float32");
    u = u.contiguous();
    check_rc(akt_kept_index_from_uniform((const float*)ptr(u), (float)*kept_ratio, rows, n, n,
                                         (const int32_t*)ptr(rl), (int32_t*)ptr(ind), l_max,
                                         (int32_t*)ptr(nnz), ensure_nonempty ? 1 : 0, st),
             "akt_kept_index_from_uniform");
  }
  return py::make_tuple(ind, nnz);
}

// The cached workspaces, as (device index, stream handle, buffer) tuples.
py::list workspaces() {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  py::list out;
  for (const auto& kv : g_ws)
    out.append(py::make_tuple(kv.first.first, (uintptr_t)kv.first.second, kv.second));
  return out;
}

}  // namespace

PYBIND11_MODULE(_akt_torch, m) {
  m.doc() = "Compiled host layer of the hot attention entry points (calls libakt_amd.so)";
  m.def("prefill", &prefill, py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("causal"),
        py::arg("softmax_scale"), py::arg("varlen") = py::none(), py::arg("return_lse") = false);
  m.def("decode", &decode, py::arg("q"), py::arg("K"), py::arg("V"), py::arg("softmax_scale"),
        py::arg("return_lse") = false, py::arg("chunk_tokens") = 0);
  m.def("decode_paged", &decode_paged, py::arg("q"), py::arg("paged_kv_cache"),
        py::arg("kv_page_indptr"), py::arg("kv_page_indices"), py::arg("kv_last_page_len"),
        py::arg("softmax_scale") = py::none(), py::arg("return_lse") = false,
        py::arg("chunk_tokens") = 0);
  m.def("sparse_decode", &sparse_decode, py::arg("q"), py::arg("K"), py::arg("V"),
        py::arg("sparse_ind"), py::arg("sparse_nnz"), py::arg("softmax_scale"),
        py::arg("return_lse") = false, py::arg("num_splits") = 0);
  m.def("sparse_decode_paged", &sparse_decode_paged, py::arg("q"), py::arg("paged_kv_cache"),
        py::arg("kv_page_indptr"), py::arg("kv_page_indices"), py::arg("sparse_ind"),
        py::arg("sparse_nnz"), py::arg("softmax_scale") = py::none(),
        py::arg("return_lse") = false, py::arg("num_splits") = 0, py::arg("lsh_k") = py::none(),
        py::arg("lsh_l") = py::none());
  m.def("kept_indices", &kept_indices, py::arg("l_max"), py::arg("mask") = py::none(),
        py::arg("uniform") = py::none(), py::arg("kept_ratio") = py::none(),
        py::arg("row_len") = py::none(), py::arg("ensure_nonempty") = true);
  m.def("workspaces", &workspaces);
}
