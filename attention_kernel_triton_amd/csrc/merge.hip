// Log-sum-exp merge of attention states (partial outputs with their LSE).
//
// Given N partial results of attention over disjoint key sets -- O_i and
// LSE_i = ln sum_{k in set i} exp(s_k) for each (query, head) row -- the
// result over the union is
//   LSE = ln sum_i exp(LSE_i),   O = sum_i exp(LSE_i - LSE) O_i.
// This is the standalone form of the combine the split-KV decode kernels
// run internally; it joins chunked prefill / decode calls or per-GPU shards.
// The reference has no such operator: its LSE stores are commented out
// (prefill_flash_attention.py:331-334, decode_flash_attention_redundant.py:225-228).
//
// Work: each thread owns 8 consecutive dims of one row and walks the parts
// once with an online max (one exp2 per part and row); rows are packed
// D / 8 threads apiece into 256-thread workgroups.  HBM-bound: bytes per row
// = N * (D * sizeof(in) + 4) + D * sizeof(out) + 4.
#include <math.h>

#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kMThreads = 256;
constexpr int kMaxMergeDim = 512;

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void load8<half_t>(const half_t* p, float (&v)[8]) {
  const half8_t h = as_half8(ld16(p));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  const float4_t a = *reinterpret_cast<const float4_t*>(p);
  const float4_t b = *reinterpret_cast<const float4_t*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]);
template <>
__device__ __forceinline__ void store8<half_t>(half_t* p, const float (&v)[8]) {
  half8_t h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];
  st16(p, as_uint4(h));
}
template <>
__device__ __forceinline__ void store8<float>(float* p, const float (&v)[8]) {
  float4_t a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = v[i];
    b[i] = v[4 + i];
  }
  *reinterpret_cast<float4_t*>(p) = a;
  *reinterpret_cast<float4_t*>(p + 4) = b;
}

struct MergeParams {
  const void* o_parts;
  const float* lse_parts;
  void* o_out;
  float* lse_out;
  int64_t n_parts, rows, D;
  int64_t o_sp, o_sr;      // parts: part / row strides (elements)
  int64_t l_sp, l_sr;      // lse parts: part / row strides
  int64_t out_sr, lse_sr;  // outputs: row strides
  int tpr;                 // threads per row (D / 8)
};

template <typename TI, typename TO>
__global__ __launch_bounds__(kMThreads) void merge_kernel(MergeParams p) {
  const int64_t gt = (int64_t)blockIdx.x * kMThreads + threadIdx.x;
  const int64_t row = gt / p.tpr;
  const int d0 = (int)(gt - row * p.tpr) * 8;
  if (row >= p.rows) return;
  const TI* op = static_cast<const TI*>(p.o_parts) + row * p.o_sr + d0;
  const float* lp = p.lse_parts + row * p.l_sr;
  // Online merge in log2 units: m = running max of LSE_i * log2(e).  Parts
  // go kBatch at a time with every load of the batch issued first (a part's
  // O is loaded whatever its LSE, so no load waits for another); an empty
  // part (LSE -inf) then has weight 0 and its O, which may hold anything, is
  // never used.
  constexpr int kBatch = 4;
  float m = -__builtin_inff(), s = 0.f, acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int64_t i0 = 0; i0 < p.n_parts; i0 += kBatch) {
    float l[kBatch], v[kBatch][8];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i = i0 + u;
      l[u] = -__builtin_inff();
      if (i < p.n_parts) {  // uniform
        l[u] = lp[i * p.l_sp] * kLog2e;
        load8<TI>(op + i * p.o_sp, v[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (l[u] == -__builtin_inff()) continue;  // empty (or absent) part: weight 0
      if (l[u] > m) {
        const float a = fast_exp2(m - l[u]);  // 0 on the first non-empty part
        s *= a;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] *= a;
        m = l[u];
      }
      const float w = fast_exp2(l[u] - m);
      s += w;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(w, v[u][j], acc[j]);
    }
  }
  const float inv = s > 0.f ? 1.0f / s : 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] *= inv;
  store8<TO>(static_cast<TO*>(p.o_out) + row * p.out_sr + d0, acc);
  if (p.lse_out && d0 == 0)
    p.lse_out[row * p.lse_sr] = s > 0.f ? (m + __log2f(s)) * kLn2 : -__builtin_inff();
}

template <typename TI, typename TO>
int launch_merge(const MergeParams& p, hipStream_t st) {
  const int64_t threads = p.rows * p.tpr;
  const int64_t grid = ceil_div(threads, kMThreads);
  AKT_CHECK(grid < (1ll << 31), "too many rows");
  KernelTimer timer;
  timer.launch(merge_kernel<TI, TO>, dim3((unsigned)grid), dim3(kMThreads), 0, st, p);
  return check_launch("merge_kernel");
}

}  // namespace
}  // namespace akt

using namespace akt;

extern "C" int akt_merge_states(const void* o_parts, int o_parts_dtype, const float* lse_parts,
                                void* o_out, int o_out_dtype, float* lse_out, int64_t n_parts,
                                int64_t rows, int64_t head_dim, const int64_t o_parts_stride[2],
                                const int64_t lse_parts_stride[2], int64_t o_out_row_stride,
                                int64_t lse_out_row_stride, void* stream) {
  clear_error();
  AKT_CHECK(n_parts >= 0 && rows >= 0, "n_parts and rows must be non-negative");
  AKT_CHECK(head_dim > 0 && head_dim % 8 == 0 && head_dim <= kMaxMergeDim,
            "head_dim must be a positive multiple of 8 up to %d, got %lld", kMaxMergeDim,
            (long long)head_dim);
  AKT_CHECK(o_parts_dtype == AKT_DTYPE_F16 || o_parts_dtype == AKT_DTYPE_F32,
            "o_parts_dtype must be AKT_DTYPE_F16 or AKT_DTYPE_F32");
  AKT_CHECK(o_out_dtype == AKT_DTYPE_F16 || o_out_dtype == AKT_DTYPE_F32,
            "o_out_dtype must be AKT_DTYPE_F16 or AKT_DTYPE_F32");
  if (rows == 0) return AKT_OK;
  AKT_CHECK(o_out && o_parts_stride && lse_parts_stride, "o_out and strides are required");
  AKT_CHECK(n_parts == 0 || (o_parts && lse_parts), "o_parts and lse_parts are required");
  const int esz_in = o_parts_dtype == AKT_DTYPE_F16 ? 2 : 4;
  const int esz_out = o_out_dtype == AKT_DTYPE_F16 ? 2 : 4;
  AKT_CHECK((n_parts == 0 || aligned16(o_parts)) && aligned16(o_out) &&
                (o_parts_stride[0] * esz_in) % 16 == 0 && (o_parts_stride[1] * esz_in) % 16 == 0 &&
                (o_out_row_stride * esz_out) % 16 == 0,
            "o_parts / o_out rows must be 16-byte aligned");
  AKT_CHECK(!lse_out || aligned4(lse_out), "lse_out must be 4-byte aligned");
  MergeParams p = {};
  p.o_parts = o_parts;
  p.lse_parts = lse_parts;
  p.o_out = o_out;
  p.lse_out = lse_out;
  p.n_parts = n_parts;
  p.rows = rows;
  p.D = head_dim;
  p.o_sp = o_parts_stride[0];
  p.o_sr = o_parts_stride[1];
  p.l_sp = lse_parts_stride[0];
  p.l_sr = lse_parts_stride[1];
  p.out_sr = o_out_row_stride;
  p.lse_sr = lse_out_row_stride;
  p.tpr = (int)(head_dim / 8);
  hipStream_t st = (hipStream_t)stream;
  if (o_parts_dtype == AKT_DTYPE_F16)
    return o_out_dtype == AKT_DTYPE_F16 ? launch_merge<half_t, half_t>(p, st)
                                        : launch_merge<half_t, float>(p, st);
  return o_out_dtype == AKT_DTYPE_F16 ? launch_merge<float, half_t>(p, st)
                                      : launch_merge<float, float>(p, st);
}
