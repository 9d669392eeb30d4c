// Split-KV decode family for gfx950.
//
// One kernel skeleton serves every single-query path of the reference:
//   dense GQA decode      decode_flash_attention_redundant.py:71-229
//   paged var-len decode  decode_flash_attention_redundant_var_len_paged.py:70-224
//   sparse-token decode   sparsetoken_decode_flash_attention_redundant.py:11-124
//   sparse paged decode   sparsetoken_decode_flash_attention_redundant_var_len_paged.py:11-167
//   MagicPIG with norm    magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm.py:16-164
//
// Work decomposition.  A "unit" is the set of query heads that read the same
// K/V rows: for dense and paged caches all (up to GT) query heads of one kv
// head (the reference instead re-reads K/V once per query head and pads the
// query to 16 rows, decode_flash_attention_redundant.py:235); for sparse paths
// one query head (each head keeps its own token set).  A unit's logical token
// sequence is cut into chunks; one 256-thread workgroup owns one chunk of one
// unit and its four waves take 16-token groups round-robin.  Each wave keeps
// an online softmax in registers, the waves are merged through LDS, and the
// workgroup writes either the final output (single-chunk units) or a partial
// (m, l, o).  The log-sum-exp combine of a unit's partials runs in the same
// launch: each partial is stored with device-scope (sc1) stores, the
// workgroup then counts itself in the unit's arrival counter, and the
// workgroup that arrives last reads every partial back with device-scope
// loads and writes the unit's output.  No L2 write-back fence is needed (the
// partials never sit dirty in one XCD's L2) and no second kernel runs.
//
// Per 16-token group a wave computes the 16 x GT score block with four (D=128)
// v_mfma_f32_16x16x32_f16: A = K rows (token = lane & 15, each lane holds a
// contiguous D/4-element slice of its row), B = q^T (head = lane & 15).  The
// result lands as S^T: lane l holds head l & 15 for tokens 4*(l >> 4) + r.
// P.V runs on the VALU with v_dot2_f32_f16 over token pairs; V is loaded so
// that each 16-lane row holds the same four tokens its score registers cover,
// which makes the probability broadcast a within-row shuffle.
#include <math.h>

#include <atomic>
#include <mutex>

#include "akt_common.hpp"
#include "akt_host.hpp"
#include "paged_stream.hpp"

namespace akt {

enum : int { kModeDense = 0, kModePaged = 1, kModeSparseDense = 2, kModeSparsePaged = 3 };

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// Split-KV chunk lengths (tokens) of dense and paged caches: 128, 256, 512 or
// 640, i.e. 2, 4, 8 or 10 16-token groups per wave.
// Largest batch whose paged chunk table fits the persistent kernel's LDS.
constexpr int kMaxTableB = 1024;
constexpr int kMaxDevices = 64;
// Workspace header holding the scheduling counters; zero between launches.
constexpr size_t kCounterBytes = 256;
// Partials are addressed with 32-bit byte offsets.
constexpr int64_t kMaxPartialBytes = (int64_t)1 << 31;
#define AKT_NEG_INF (-__builtin_inff())

struct SplitParams {
  const half_t* q;
  const half_t* kbase;  // dense: K tensor; paged: KV pool
  const half_t* vbase;  // dense: V tensor; paged: KV pool + stride of the K/V axis
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  const int32_t* sparse_ind;
  const int32_t* sparse_nnz;
  const int64_t* csr_ptr;  // CSR kept-index rows: row u = sparse_ind[csr_ptr[u] .. csr_ptr[u+1])
  const float* lsh_k;
  const float* lsh_l;
  half_t* o;      // [B, Hq, D] contiguous
  float* lse;     // [B, Hq] or null
  int* counters;  // [2]: work tickets, exited workgroups (zero between launches)
  int* arrive;    // [units]: partials stored so far per unit (zero between launches)
  float* part_o;  // [parts, GT, D]
  float* part_ml; // [parts, GT, 4]: running max, fp16-P normaliser, fp32 normaliser, pad
  int64_t q_sb, q_sh;
  // Row address of a K/V row = base + row_a * s_a + row_b * s_b + unit offset.
  // dense: row_a = token, unit offset = b*s_batch + kvh*s_head.
  // paged: row_a = page id, row_b = slot, unit offset = kvh*s_head.
  int64_t k_sa, k_sb, k_batch, k_head;
  int64_t v_sa, v_sb, v_batch, v_head;
  int64_t ind_sb, ind_sh, nnz_sb, nnz_sh;
  int B, Hq, Hkv, G;
  int S;             // dense / sparse-dense: cache length
  int page_size;
  int num_pool_pages;
  int l_max;
  int n_hg;          // head groups per kv head (dense / paged)
  int chunk;         // tokens per chunk (dense / paged), multiple of 64
  int n_split;       // chunks per unit (sparse)
  float qk_scale;    // softmax_scale * log2(e)
  float inv_sqrt_d;  // 1 / sqrt(head_dim) (MagicPIG)
};

__device__ __forceinline__ int paged_len(const int32_t* __restrict__ indptr,
                                         const int32_t* __restrict__ last_len, int b, int P) {
  int np = indptr[b + 1] - indptr[b];
  if (np <= 0) return 0;
  int ll = min(max(last_len[b], 0), P);
  return (np - 1) * P + ll;
}

// Wave-cooperative: find the sequence that owns global chunk x, where sequence
// b owns ceil(len_b / chunk) consecutive chunks.  Returns false if x is past
// the last chunk.
__device__ bool locate_chunk(const SplitParams& p, int x, int& b_out, int& c_out, int& nch_out,
                             int& len_out) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int bb = base + lane;
    int len = 0, n = 0;
    if (bb < p.B) {
      len = paged_len(p.indptr, p.last_len, bb, p.page_size);
      n = (len + p.chunk - 1) / p.chunk;
    }
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const int start = carry + incl - n;
    const bool hit = (n > 0) && (x >= start) && (x < start + n);
    const uint64_t m = __ballot(hit);
    if (m) {
      const int src = __builtin_ctzll(m);
      b_out = base + src;
      c_out = x - __shfl(start, src, 64);
      nch_out = __shfl(n, src, 64);
      len_out = __shfl(len, src, 64);
      return true;
    }
    carry += __shfl(incl, 63, 64);
  }
  return false;
}

// g(y) = log1p(y) - y for y > -1, without the cancellation of the direct
// difference near 0.  With s = y / (2 + y), log1p(y) = 2 atanh(s) =
// 2 (s + s^3/3 + s^5/5 + ...) and 2 s - y = -y s, so
//   g(y) = -y s + 2 s^3 (1/3 + s^2/5 + s^4/7 + s^6/9 + s^8/11 + ...),
// whose two parts never cancel for |y| < 0.25 (|s| < 1/7: the dropped terms
// are below 1e-10 relative).  From |y| = 0.25 on, the direct difference
// loses at most 3 bits.
__device__ __forceinline__ float log1p_minus_id(float y) {
  if (fabsf(y) < 0.25f) {
    const float s = y / (2.0f + y);
    const float s2 = s * s;
    const float poly =
        (1.0f / 3.0f) + s2 * ((1.0f / 5.0f) + s2 * ((1.0f / 7.0f) + s2 * ((1.0f / 9.0f) + s2 * (1.0f / 11.0f))));
    return __builtin_fmaf(-y, s, 2.0f * s * s2 * poly);
  }
  return log1pf(y) - y;
}

// MagicPIG correction ln u for one token (eq. 11 of the reference's
// attention_with_norm.png, as evaluated in
// magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm.py:110-160):
//   p = 1 - acos(c) / pi (clamped to [0, 1]),  x = p^K,
//   u = 1 - (1 - x)^L - L x (1 - x)^(L - 1),  clamped to >= 1e-10.
// u is a difference of nearly equal terms when x is small or L is near 1, so
// it is evaluated in fp32 in a form without that cancellation.  With m = L - 1,
//   u = 1 - (1 - x)^m (1 + m x) = -expm1(f),
//   f = m log1p(-x) + log1p(m x) = m g(-x) + g(m x),   g(y) = log1p(y) - y
// (the linear terms -m x and +m x cancel exactly), and for L >= 1 both parts
// of f are <= 0, so nothing cancels for any x in [0, 1) and any L >= 1.  The
// relative error of u stays within a few fp32 ulps.  Outside that domain
// (x >= 1 from K < 0, or m x <= -1 from L < 0) the reference's formula is
// evaluated as written, with its clamp of 1 - x to [0, 1].
__device__ __forceinline__ float magicpig_log_u(float cosv, float K, float L) {
  const float pp = fminf(fmaxf(1.0f - acosf(cosv) * (float)M_1_PI, 0.0f), 1.0f);
  const float x = pp > 0.0f ? __expf(K * __logf(pp)) : 0.0f;
  const float m = L - 1.0f;
  const float mx = m * x;
  float u;
  if (x < 1.0f && mx > -1.0f) {
    u = -expm1f(__builtin_fmaf(m, log1p_minus_id(-x), log1p_minus_id(mx)));
  } else {
    const float om = fminf(fmaxf(1.0f - x, 0.0f), 1.0f);
    u = 1.0f - powf(om, L) - L * x * powf(om, m);
  }
  return __logf(fmaxf(u, 1e-10f));
}

// ---------------------------------------------------------------------------
// Split kernel.
// ---------------------------------------------------------------------------
// Resolved work item: a chunk [t0, t1) of one unit (wave-uniform values).
// The unit's chunks c = 0 .. nch - 1 keep their partials at partial index
// pfirst + c * pstep; pidx is this item's.
struct Item {
  int b, kvh, hq0, nh, t0, t1, pstart, np, direct;
  int nch, unit, pstep;
  int64_t pidx, pfirst;
  int64_t ind_off;  // sparse: offset of the unit's kept-index row in sparse_ind
};

// Everything needed to issue the loads of one item's groups.
struct IssueCtx {
  const half_t* kb;  // K base of the unit (dense: + batch/head offset; paged: + head offset)
  const half_t* vb;
  int64_t k_dummy, v_dummy;  // offsets of the unit's q row from kb / vb
  const int* ind_row;        // sparse: kept-index row
  int t1, g_begin, pstart, np;
  int page_pref, slot_pref;  // aligned paged: page id / slot of this wave's k-th group (lane k)
};

// PERSIST: the grid is sized to the machine and each workgroup starts with
// item blockIdx.x and takes the rest from a ticket counter (dense and paged
// caches; see the driver below).  For a
// paged cache the per-sequence chunk prefix is built once per workgroup in
// LDS, so resolving an item needs no global loads.  Each wave streams its
// groups continuously across items: the last two groups of an item are
// followed by the first two of the next, issued before the item's
// workgroup merge, so the memory pipeline never drains between items.
// Otherwise (sparse units) one workgroup handles the item named by blockIdx.
// Two workgroups per CU (two waves per SIMD) is what hides a unit's load
// latency; instances whose state fits in 256 registers per lane are held to it.
template <int D, int GT>
constexpr int split_min_waves() {
  return (D <= 128 && GT <= 4) ? 2 : 1;
}

template <int D, int GT, int MODE, bool ALIGNED, bool MAGIC, int GPW, bool PERSIST>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(split_min_waves<D, GT>(), 8))) void split_kernel(SplitParams p) {
  constexpr int KPL = D / 4;                 // K elements per lane per group
  constexpr int KS = D / 32;                 // MFMA k-steps (8 elements each)
  constexpr int VTOK = (D == 64) ? 2 : 4;    // V tokens per lane per group
  constexpr int VDIM = (D == 256) ? 16 : 8;  // V dims per lane
  constexpr int VLD = VDIM / 8;              // 16-byte loads per V token
  constexpr int NPAIR = VTOK / 2;
  constexpr bool SPARSE = (MODE == kModeSparseDense || MODE == kModeSparsePaged);
  constexpr bool PAGED_ADDR = (MODE == kModePaged || MODE == kModeSparsePaged);
  static_assert(!SPARSE || GT == 1, "sparse units hold one query head");
  static_assert(SPARSE == (GPW == 0), "sparse units have a dynamic group count");
  static_assert(!SPARSE || !PERSIST, "sparse units are not persistent");
  static_assert(GPW == 0 || GPW >= 2, "the cross-item pipeline needs two groups per wave");
  constexpr bool TABLE = PERSIST && MODE == kModePaged;

  __shared__ __attribute__((aligned(16))) float sm_o[kWaves][GT][D];
  __shared__ float sm_m[kWaves][GT];
  __shared__ float sm_l[kWaves][GT];
  __shared__ float sm_e[kWaves][GT];
  __shared__ int sm_last;   // this workgroup stored the unit's last partial
  __shared__ int sm_pflag;  // ... of the pending item's unit (persistent loop)
  __shared__ Item sm_pend;  // the pending item (persistent loop; written by thread 0)
  // Paged persistent: chunk prefix, length and first page of every sequence.
  __shared__ int sm_cs[TABLE ? kMaxTableB + 1 : 1];
  __shared__ int sm_len[TABLE ? kMaxTableB : 1];
  __shared__ int sm_ps[TABLE ? kMaxTableB : 1];
  __shared__ int sm_wtot[kWaves];
  __shared__ int sm_next;
  // The next item's ticket (low word) and the count of items whose ticket
  // thread 0 has published (high word), written and read as one word.
  __shared__ unsigned long long sm_tick;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);  // wave-uniform: keeps group math in SGPRs
  const int R = lane >> 4;
  const int c16 = lane & 15;
  const int Y = p.Hkv * p.n_hg;  // units per chunk index (dense / paged)
  const uint32_t kOnes = 0x3c003c00u;  // half2(1, 1)

  // ---- work item resolution ----------------------------------------------
  auto finish_item = [&](Item& w, int x, int y, int c, int nch, int len) {
    w.kvh = y / p.n_hg;
    const int hg = y - w.kvh * p.n_hg;
    w.hq0 = w.kvh * p.G + hg * GT;
    w.nh = min(GT, p.G - hg * GT);
    w.t0 = c * p.chunk;
    w.t1 = min(len, w.t0 + p.chunk);
    w.pidx = (int64_t)x * Y + y;
    w.direct = (nch == 1);
    w.nch = nch;
    w.unit = w.b * Y + y;
    w.pfirst = (int64_t)(x - c) * Y + y;  // chunk x - c is the sequence's first
    w.pstep = Y;
  };
  // Item i of the persistent order: chunk index x = i / Y, unit y = i % Y.
  auto resolve_persistent = [&](int i) -> Item {
    Item w = {};
    const int x = i / Y;
    const int y = i - x * Y;
    if constexpr (MODE == kModeDense) {
      const int nch = (p.S + p.chunk - 1) / p.chunk;
      w.b = x / nch;
      finish_item(w, x, y, x - w.b * nch, nch, p.S);
    } else if constexpr (TABLE) {
      int lo = 0, hi = p.B - 1;  // last sequence whose first chunk is <= x
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sm_cs[mid] <= x) lo = mid;
        else hi = mid - 1;
      }
      w.b = lo;
      w.pstart = sm_ps[lo];
      w.np = (sm_len[lo] + p.page_size - 1) / p.page_size;
      finish_item(w, x, y, x - sm_cs[lo], sm_cs[lo + 1] - sm_cs[lo], sm_len[lo]);
    }
    return w;
  };
  auto resolve_block = [&]() -> Item {
    Item w = {};
    if constexpr (MODE == kModePaged) {
      int c, nch, len;
      if (!locate_chunk(p, blockIdx.x, w.b, c, nch, len)) {
        w.b = -1;
        return w;
      }
      finish_item(w, blockIdx.x, blockIdx.y, c, nch, len);
      w.pstart = p.indptr[w.b];
      w.np = p.indptr[w.b + 1] - w.pstart;
    } else if constexpr (SPARSE) {
      // Block x is split c = x / rows of row u = x % rows: consecutive blocks,
      // which the dispatcher deals to the XCDs in turn, are different rows,
      // so that the splits of one row (and the short last splits) spread
      // over the XCDs.
      const int x = blockIdx.x;
      const int rows = (int)gridDim.x / p.n_split;
      const int c = x / rows;
      const int u = x - c * rows;
      w.b = u / p.Hq;
      w.hq0 = u - w.b * p.Hq;
      w.kvh = w.hq0 / p.G;
      w.nh = 1;
      int n;
      if (p.csr_ptr) {  // CSR rows: any length, no padding
        const int64_t r0 = p.csr_ptr[u], r1 = p.csr_ptr[u + 1];
        w.ind_off = r0;
        n = (int)min(max(r1 - r0, (int64_t)0), (int64_t)INT32_MAX);
      } else {  // padded rows [B, Hq, l_max] with a count per row
        w.ind_off = (int64_t)w.b * p.ind_sb + (int64_t)w.hq0 * p.ind_sh;
        n = p.sparse_nnz[(int64_t)w.b * p.nnz_sb + (int64_t)w.hq0 * p.nnz_sh];
        n = min(max(n, 0), p.l_max);
        // A dense-cache row with no kept token attends to its first index
        // slot, as the reference's PyTorch path does (it treats nnz == 0 as
        // nnz == 1, sparsetoken_decode_flash_attention_redundant.py:191-194);
        // with the harness's -1 padding that slot names the last row.
        if constexpr (MODE == kModeSparseDense) n = max(n, min(1, p.l_max));
      }
      // Split c covers [c*per, min(n, (c+1)*per)); per is a multiple of 16 so
      // every split starts on a 16-token group and splits never share a group.
      const int per = ((n + p.n_split - 1) / p.n_split + 15) & ~15;
      w.t0 = c * per;
      w.t1 = max(w.t0, min(n, w.t0 + per));
      w.pidx = (int64_t)u * p.n_split + c;
      w.direct = (p.n_split == 1);
      w.nch = p.n_split;
      w.unit = u;
      w.pfirst = (int64_t)u * p.n_split;
      w.pstep = 1;
      if constexpr (MODE == kModeSparsePaged) {
        w.pstart = p.indptr[w.b];
        w.np = p.indptr[w.b + 1] - w.pstart;
      }
    }
    return w;
  };
  // The work item is wave-uniform; say so, so that the group loop and all
  // per-group address math stay scalar.
  auto make_uniform = [&](Item& w) {
    w.b = uniform(w.b);
    w.kvh = uniform(w.kvh);
    w.hq0 = uniform(w.hq0);
    w.nh = uniform(w.nh);
    w.t0 = uniform(w.t0);
    w.t1 = uniform(w.t1);
    w.pstart = uniform(w.pstart);
    w.np = uniform(w.np);
    w.direct = uniform(w.direct);
    w.nch = uniform(w.nch);
    w.unit = uniform(w.unit);
    w.pstep = uniform(w.pstep);
  };

  // ---- per-item setup: issue context (with page prefetch) and q fragment ----
  // Query fragment (B operand): head hq0 + c16, dims R*KPL + 8s + e.  For paged
  // caches with page_size % 16 == 0 (one page per 16-token group), lane k
  // prefetches the page id and slot of this wave's k-th group (a chunk has at
  // most kMaxChunk tokens, so at most 10 groups per wave).
  auto setup = [&](const Item& w, IssueCtx& cx, half8_t (&qd)[KS]) {
    const int64_t k_unit = PAGED_ADDR ? (int64_t)w.kvh * p.k_head
                                      : (int64_t)w.b * p.k_batch + (int64_t)w.kvh * p.k_head;
    const int64_t v_unit = PAGED_ADDR ? (int64_t)w.kvh * p.v_head
                                      : (int64_t)w.b * p.v_batch + (int64_t)w.kvh * p.v_head;
    cx.kb = p.kbase + k_unit;
    cx.vb = p.vbase + v_unit;
    const half_t* qrow0 = p.q + (int64_t)w.b * p.q_sb + (int64_t)w.hq0 * p.q_sh;
    cx.k_dummy = qrow0 - cx.kb;
    cx.v_dummy = qrow0 - cx.vb;
    cx.ind_row = nullptr;
    if constexpr (SPARSE)
      cx.ind_row = p.sparse_ind + w.ind_off;
    cx.t1 = w.t1;
    cx.g_begin = w.t0 >> 4;
    cx.pstart = w.pstart;
    cx.np = w.np;
    cx.page_pref = 0;
    cx.slot_pref = 0;
    if constexpr (MODE == kModePaged && ALIGNED) {
      const int g_end = (w.t1 + 15) >> 4;
      const int gk = cx.g_begin + wave + kWaves * lane;
      // Clamped into the item (an empty one keeps g_begin): the load is
      // issued unconditionally.
      const int gc = max(min(gk, g_end - 1), cx.g_begin);
      const int lp = (gc << 4) / p.page_size;
      cx.page_pref = p.indices[w.pstart + lp];
      cx.slot_pref = (gc << 4) - lp * p.page_size;
    }
    const bool hv = c16 < w.nh;
    const half_t* qrow = qrow0 + (int64_t)(hv ? c16 : 0) * p.q_sh + R * KPL;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4_t v = ld16(qrow + 8 * s);
      if (!hv) v = uint4_t{0, 0, 0, 0};
      qd[s] = as_half8(v);
    }
  };

  // One 16-token group in flight: its K slice, V rows and usable-token mask.
  struct Buf {
    uint4_t k[KS];
    uint4_t v[VTOK][VLD];
    uint32_t vmask;
  };

  // Computes the row addresses of group g and issues its K/V loads.  Every
  // load is issued unconditionally (a lane whose token is unusable reads the
  // unit's own q row instead, which is always mapped and finite) so that no
  // load sits behind a branch: the wait counts then only cover the buffer
  // being consumed.  Index and page lookups read clamped, in-range entries.
  // Paged caches of whole 16-token groups: a group is the 16 rows from row
  // `slot` of one page (uniform), so each of its addresses is a uniform base
  // plus a per-lane byte offset that is the same for every group: this lane's
  // K row (c16) and K slice (R), and its V token (4R + i, or for D = 64
  // 4R + 2 (c16 / 8) + i, plus v_sb bytes per i) at dims dim0.
  const int dim0 = (D == 64) ? 8 * (c16 & 7) : VDIM * c16;
  const int tt0 = (D == 64) ? (4 * R + 2 * (c16 >> 3)) : 4 * R;
  uint32_t lane_kofs = 0, lane_qofs = 0, lane_v0ofs = 0, lane_dofs = 0;
  if constexpr (MODE == kModePaged && ALIGNED) {
    lane_kofs = (uint32_t)(c16 * (int)p.k_sb + R * KPL) * 2u;
    lane_qofs = (uint32_t)(R * KPL) * 2u;
    lane_v0ofs = (uint32_t)(tt0 * (int)p.v_sb + dim0) * 2u;
    lane_dofs = (uint32_t)dim0 * 2u;
  }
  auto issue = [&](const IssueCtx& cx, int g, Buf& bf) {
    const int t1 = cx.t1;
    const int gpos = g << 4;
    if constexpr (MODE == kModePaged && ALIGNED) {
      // The usable tokens of the group are a prefix (positions below t1 of
      // a valid page).  K rows past it lie inside the page and load as they
      // are (their scores are masked); the V rows of unusable tokens re-read
      // the group's first row, a usable token whenever the group has one; a
      // group without usable tokens (or with an invalid page id) reads the
      // unit's q row instead, which is always mapped and finite.
      const int k = (g - cx.g_begin - wave) / kWaves;
      const int page = __builtin_amdgcn_readlane(cx.page_pref, k);
      const int gslot = __builtin_amdgcn_readlane(cx.slot_pref, k);
      const bool page_ok = page >= 0 && page < p.num_pool_pages;
      const int nvalid = page_ok ? min(max(t1 - gpos, 0), 16) : 0;
      bf.vmask = (uint32_t)((1u << nvalid) - 1u);
      const char* kg = reinterpret_cast<const char*>(
          page_ok ? cx.kb + (int64_t)page * p.k_sa + (int64_t)gslot * p.k_sb : cx.kb + cx.k_dummy);
      const uint32_t ko = page_ok ? lane_kofs : lane_qofs;
#pragma unroll
      for (int s = 0; s < KS; ++s) bf.k[s] = ld16(kg + ko + 16 * s);
      const char* vg = reinterpret_cast<const char*>(
          nvalid > 0 ? cx.vb + (int64_t)page * p.v_sa + (int64_t)gslot * p.v_sb
                     : cx.vb + cx.v_dummy);
      const uint32_t vstep = (uint32_t)p.v_sb * 2u;
#pragma unroll
      for (int i = 0; i < VTOK; ++i) {
        const uint32_t vo = tt0 + i < nvalid ? lane_v0ofs + (uint32_t)i * vstep : lane_dofs;
#pragma unroll
        for (int j = 0; j < VLD; ++j) bf.v[i][j] = ld16(vg + vo + 16 * j);
      }
      return;
    }
    const int pos_k = gpos + c16;
    int ra = 0, rb = 0;
    bool kval = pos_k < t1;
    if constexpr (MODE == kModeDense) {
      ra = pos_k;
    } else if constexpr (MODE == kModePaged) {
      const int pc = min(pos_k, t1 - 1);  // t1 <= len, so pc's page is in the table
      const int lp = pc / p.page_size;
      const int page = p.indices[cx.pstart + lp];
      kval = kval && page >= 0 && page < p.num_pool_pages;
      ra = page;
      rb = pc - lp * p.page_size;
    } else if constexpr (MODE == kModeSparseDense) {
      int t = cx.ind_row[min(pos_k, t1 - 1)];
      // Indices follow torch indexing, as the reference's gather K[b, h, ind]
      // does (sparsetoken_decode_flash_attention_redundant.py:196): -S <= t < 0
      // names row S + t.
      if (t < 0) t += p.S;
      kval = kval && t >= 0 && t < p.S;
      ra = t;
    } else {  // sparse paged
      const int t = cx.ind_row[min(pos_k, t1 - 1)];
      const int lp = t >= 0 ? t / p.page_size : 0;
      kval = kval && t >= 0 && lp < cx.np;
      // np == 0 (no pages) reads the unit's first kept index (always mapped)
      // instead of an empty page table; such tokens are never used.
      const int* pptr = cx.np > 0 ? p.indices + cx.pstart + min(lp, cx.np - 1) : cx.ind_row;
      const int page = *pptr;
      kval = kval && page >= 0 && page < p.num_pool_pages;
      ra = page;
      rb = t - lp * p.page_size;
    }
    const uint32_t vmask = (uint32_t)__ballot(kval) & 0xffffu;  // bit t: token gpos + t usable
    bf.vmask = vmask;
    {
      const int64_t off = (int64_t)ra * p.k_sa + (int64_t)rb * p.k_sb;
      const half_t* kr = cx.kb + (kval ? off : cx.k_dummy) + R * KPL;
#pragma unroll
      for (int s = 0; s < KS; ++s) bf.k[s] = ld16(kr + 8 * s);
    }
#pragma unroll
    for (int i = 0; i < VTOK; ++i) {
      const int tt = tt0 + i;
      const bool vv = (vmask >> tt) & 1;
      int va, vbb;
      if constexpr (MODE == kModeDense) {
        va = gpos + tt;
        vbb = 0;
      } else {
        va = __shfl(ra, tt, 64);
        vbb = __shfl(rb, tt, 64);
      }
      const int64_t off = (int64_t)va * p.v_sa + (int64_t)vbb * p.v_sb;
      const half_t* vr = cx.vb + (vv ? off : cx.v_dummy) + dim0;
#pragma unroll
      for (int j = 0; j < VLD; ++j) bf.v[i][j] = ld16(vr + 8 * j);
    }
  };

  // ---- per-item accumulation state ----------------------------------------
  Item it;
  half8_t qf[KS];
  float q_norm = 0.f, lsh_k = 0.f, lsh_l = 0.f;  // MagicPIG
  float m_run;   // running max of head c16 (log2 units)
  // Partial normalisers over this lane's tokens: l_part sums the fp16-rounded
  // probabilities that multiply V (so O is normalised consistently), e_part
  // the fp32 probabilities (for the log-sum-exp output).
  float l_part, e_part;
  float acc[GT][VDIM];

  auto begin_item = [&]() {
    m_run = AKT_NEG_INF;
    l_part = 0.f;
    e_part = 0.f;
#pragma unroll
    for (int h = 0; h < GT; ++h)
#pragma unroll
      for (int d = 0; d < VDIM; ++d) acc[h][d] = 0.f;
    if constexpr (MAGIC) {
      // |q|^2 of the unit's head (valid in lanes with c16 == 0).
      float qs = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        uint4_t u = as_uint4(qf[s]);
#pragma unroll
        for (int j = 0; j < 4; ++j) qs = dot2(u[j], u[j], qs);
      }
      q_norm = sqrtf(rows_sum(qs));
      lsh_k = p.lsh_k[(int64_t)it.b * p.Hq + it.hq0];
      lsh_l = p.lsh_l[(int64_t)it.b * p.Hq + it.hq0];
    }
  };

  // Scores, online softmax and P.V for a loaded group of the current item.
  auto consume = [&](const Buf& bf) {
    const uint32_t vmask = bf.vmask;
    float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) sacc = mfma16x16x32(as_half8(bf.k[s]), qf[s], sacc);

    float t[4];
    if constexpr (MAGIC) {
      // A sparse unit is one head (column 0 of the score tile), so the group
      // needs 16 corrections, one per token: lane l evaluates token l & 15
      // (its dot product comes from lane 16 (tt / 4), register tt % 4, and
      // |k|^2 from the K-lane layout), and each score lane then fetches the
      // scores of its tokens 4R + r.  Lanes of columns past the head carry
      // head 0's scores, which are never stored.
      float ks = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) ks = dot2(bf.k[s][j], bf.k[s][j], ks);
      ks = rows_sum(ks);
      const int tt = lane & 15;
      const int src = (tt >> 2) << 4;
      const float d0 = __shfl(sacc[0], src, 64), d1 = __shfl(sacc[1], src, 64);
      const float d2 = __shfl(sacc[2], src, 64), d3 = __shfl(sacc[3], src, 64);
      const int rr = tt & 3;
      const float dotp = rr == 0 ? d0 : (rr == 1 ? d1 : (rr == 2 ? d2 : d3));
      const float kn = sqrtf(__shfl(ks, tt, 64));
      const float qn = __shfl(q_norm, 0, 64);  // |q| of the unit's head (lane 0)
      float cosv = dotp / (qn * kn + 1e-8f);
      cosv = fminf(fmaxf(cosv, -1.0f + 1e-7f), 1.0f - 1e-7f);
      const float sc_t = dotp * p.inv_sqrt_d - magicpig_log_u(cosv, lsh_k, lsh_l);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sc = __shfl(sc_t, 4 * R + r, 64);
        t[r] = ((vmask >> (4 * R + r)) & 1) ? sc * kLog2e : AKT_NEG_INF;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        t[r] = ((vmask >> (4 * R + r)) & 1) ? sacc[r] * p.qk_scale : AKT_NEG_INF;
    }

    // online softmax (head c16)
    float mt = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
    mt = rows_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (__any(m_new > m_run)) {
      const float alpha = (m_new > m_run) ? fast_exp2(m_run - m_new) : 1.0f;
      l_part *= alpha;
      e_part *= alpha;
#pragma unroll
      for (int h = 0; h < GT; ++h) {
        const float ah = shfl_f(alpha, (lane & 48) | h);
#pragma unroll
        for (int d = 0; d < VDIM; ++d) acc[h][d] *= ah;
      }
      m_run = m_new;
    }
    const float m_use = (m_run == AKT_NEG_INF) ? 0.f : m_run;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(t[r] - m_use);
    const uint32_t p01 = pack_half2(pr[0], pr[1]);
    const uint32_t p23 = pack_half2(pr[2], pr[3]);
    l_part = dot2(p23, kOnes, dot2(p01, kOnes, l_part));
    e_part += (pr[0] + pr[1]) + (pr[2] + pr[3]);

    // P.V
    uint32_t vp[NPAIR][VDIM];
#pragma unroll
    for (int q2 = 0; q2 < NPAIR; ++q2)
#pragma unroll
      for (int j = 0; j < VLD; ++j)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t a = bf.v[2 * q2][j][w], bq = bf.v[2 * q2 + 1][j][w];
          vp[q2][8 * j + 2 * w] = pair_lo(a, bq);
          vp[q2][8 * j + 2 * w + 1] = pair_hi(a, bq);
        }
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      const int src = (lane & 48) | h;
      const uint32_t pa = shfl_u(p01, src);
      const uint32_t pb = shfl_u(p23, src);
#pragma unroll
      for (int q2 = 0; q2 < NPAIR; ++q2) {
        uint32_t pp;
        if constexpr (D == 64) pp = (c16 >> 3) ? pb : pa;
        else pp = q2 ? pb : pa;
#pragma unroll
        for (int d = 0; d < VDIM; ++d) acc[h][d] = dot2(pp, vp[q2][d], acc[h][d]);
      }
    }
  };

  // ---- output of a unit ----------------------------------------------------
  constexpr int NV = GT * D / 4;  // float4 vectors of a unit's output (head-major)
  // Groups in flight per wave in the persistent loop: 4 for dense D = 64
  // (a group's buffer is 17 registers, and a workgroup streams a single
  // item there, so the loads of a deeper window shorten its dependent chain),
  // else 2.
  constexpr int PD = (PERSIST && MODE == kModeDense && D == 64 && GPW >= 5) ? 4 : 2;
  // Arrival of a stored partial is counted one item late in the persistent
  // loop (see the driver), which needs the item's group PD (the first whose
  // loads the item itself issues).
  constexpr bool DEFER = PERSIST && GPW >= PD + 1;
  // Normalised output of head h of item w, dims d0 .. d0 + 3, and (d0 == 0) its LSE.
  auto write_out = [&](const Item& w, int h, int d0, float4_t O, float M, float L, float E) {
    const int64_t row = (int64_t)w.b * p.Hq + w.hq0 + h;
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    half4_t hv;
#pragma unroll
    for (int r = 0; r < 4; ++r) hv[r] = (half_t)(O[r] * inv);
    *reinterpret_cast<half4_t*>(p.o + row * D + d0) = hv;
    if (d0 == 0 && p.lse) p.lse[row] = E > 0.f ? (M + log2f(E)) * kLn2 : AKT_NEG_INF;
  };

  // Log-sum-exp merge of the nch partials of item w's unit, run by the
  // workgroup that counted the last of them.  A thread owns one float4 of one
  // head's output and walks its chunk group's chunks c = cg, cg + NG, ...
  // with an online max, U chunks per round trip of device-scope loads; the
  // chunk groups are then merged through LDS.  Called by every thread after a
  // barrier that follows the last read of the merge buffers.
  auto merge_unit = [&](const Item& w) {
    constexpr int NG = NV >= kThreads ? 1 : (kThreads / NV < kWaves ? kThreads / NV : kWaves);
    constexpr int U = 8;
    const int nch = w.nch;
    auto combine = [](float& M, float& L, float& E, float4_t& A, float m, float l, float e,
                      float4_t a) {
      if (m == AKT_NEG_INF) return;
      if (m > M) {
        const float s = fast_exp2(M - m);  // 0 while M = -inf (A, L, E are 0 then)
        A *= s;
        L *= s;
        E *= s;
        M = m;
      }
      const float f = fast_exp2(m - M);
      A += f * a;
      L += f * l;
      E += f * e;
    };
    auto accumulate = [&](int vec, int cg, float& M, float& L, float& E, float4_t& A) {
      const int h = (vec * 4) / D;
      const int d0 = vec * 4 - h * D;
      M = AKT_NEG_INF;
      L = E = 0.f;
      A = float4_t{0.f, 0.f, 0.f, 0.f};
      for (int c0 = cg; c0 < nch; c0 += U * NG) {
        float4_t ml[U], ov[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = min(c0 + u * NG, nch - 1);
          const int64_t ph = (w.pfirst + (int64_t)c * w.pstep) * GT + h;
          ml[u] = as_float4u(ld16_device(p.part_ml, (uint32_t)(ph * 16)));
          ov[u] = as_float4u(ld16_device(p.part_o, (uint32_t)((ph * D + d0) * 4)));
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (c0 + u * NG < nch) combine(M, L, E, A, ml[u][0], ml[u][1], ml[u][2], ov[u]);
      }
    };
    if constexpr (NG == 1) {
      for (int vec = tid; vec < NV; vec += kThreads) {
        float M, L, E;
        float4_t A;
        accumulate(vec, 0, M, L, E, A);
        const int h = (vec * 4) / D;
        if (h < w.nh) write_out(w, h, vec * 4 - h * D, A, M, L, E);
      }
    } else {
      const int vec = tid % NV;
      const int cg = tid / NV;
      const int h = (vec * 4) / D;
      const int d0 = vec * 4 - h * D;
      float M = AKT_NEG_INF, L = 0.f, E = 0.f;
      float4_t A = {0.f, 0.f, 0.f, 0.f};
      if (cg < NG) accumulate(vec, cg, M, L, E, A);
      float4_t* red = reinterpret_cast<float4_t*>(&sm_o[0][0][0]);  // [NG - 1][NV]
      if (cg >= 1 && cg < NG) {
        red[(cg - 1) * NV + vec] = A;
        if (d0 == 0) {
          sm_m[cg][h] = M;
          sm_l[cg][h] = L;
          sm_e[cg][h] = E;
        }
      }
      __syncthreads();
      if (cg == 0) {
#pragma unroll
        for (int g2 = 1; g2 < NG; ++g2)
          combine(M, L, E, A, sm_m[g2][h], sm_l[g2][h], sm_e[g2][h], red[(g2 - 1) * NV + vec]);
        if (h < w.nh) write_out(w, h, d0, A, M, L, E);
      }
    }
  };

  // Counts item w's stored partial in its unit's arrival counter (thread 0)
  // and returns, to every thread, whether this workgroup stored the unit's
  // last partial; the last one also resets the counter for the next launch.
  // Every thread first waits for its outstanding memory operations, so wave
  // 0's partial stores are complete (visible device-wide) before the count.
  auto arrive_now = [&](const Item& w) -> bool {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int prev = atomicAdd(&p.arrive[w.unit], 1);
      const int last = prev == w.nch - 1;
      if (last) atomicExch(&p.arrive[w.unit], 0);
      sm_last = last;
    }
    __syncthreads();
    return sm_last != 0;
  };

  // Persistent (DEFER) arrival state: sm_pend is the item whose partial was
  // stored at the previous finish() and is counted by thread 0 during the
  // current item (arr holds the counter's old value).  It lives in LDS: only
  // thread 0 and the rare merge read it, and registers are the scarce resource.
  bool has_pend = false;
  int arr = -1;

  // Wave reduction, workgroup merge and output of the current item; returns
  // the ticket thread 0 published in sm_next before the call.  A multi-chunk
  // item's partial is stored by wave 0 alone (so one wave's memory ordering
  // covers all of it) with device-scope stores.  Without DEFER the workgroup
  // then counts it at once and merges the unit if it was last.  With DEFER it
  // becomes sm_pend, and the previous pending item, counted during this item,
  // is merged here if this workgroup stored its unit's last partial (sm_pflag).
  auto finish = [&]() -> int {
    const float l_wave = rows_sum(l_part);
    const float e_wave = rows_sum(e_part);
#pragma unroll
    for (int h = 0; h < GT; ++h)
#pragma unroll
      for (int d = 0; d < VDIM; ++d) {
        float v = acc[h][d];
        if constexpr (D == 64) v += shfl_xor_f(v, 8);
        acc[h][d] = rows_sum(v);
      }
    if (R == 0) {
      const bool owner = (D == 64) ? (c16 < 8) : true;
      if (owner) {
        const int dim0 = (D == 64) ? 8 * c16 : VDIM * c16;
#pragma unroll
        for (int h = 0; h < GT; ++h)
#pragma unroll
          for (int d = 0; d < VDIM; ++d) sm_o[wave][h][dim0 + d] = acc[h][d];
      }
      if (c16 < GT) {
        sm_m[wave][c16] = m_run;
        sm_l[wave][c16] = l_wave;
        sm_e[wave][c16] = e_wave;
      }
    }
    __syncthreads();
    // Thread 0 wrote the next ticket (and the pending item's count) before
    // the barrier above; every wave reads them before the last barrier below,
    // so thread 0 cannot overwrite them while a wave still has to read them.
    const int next_ticket = sm_next;
    const bool merge_pend = DEFER && has_pend && sm_pflag != 0;
    const float4_t* sm_o4 = reinterpret_cast<const float4_t*>(&sm_o[0][0][0]);
    auto wave_merge = [&](int vec, float& M, float& L, float& E, float4_t& O) {
      const int h = (vec * 4) / D;
      M = AKT_NEG_INF;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
      L = E = 0.f;
      O = float4_t{0.f, 0.f, 0.f, 0.f};
      if (M != AKT_NEG_INF) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float f = fast_exp2(sm_m[w][h] - M);
          L += f * sm_l[w][h];
          E += f * sm_e[w][h];
          O += f * sm_o4[w * NV + vec];
        }
      }
    };
    if (it.direct) {
      for (int vec = tid; vec < NV; vec += kThreads) {
        const int h = (vec * 4) / D;
        if (h >= it.nh) continue;
        float M, L, E;
        float4_t O;
        wave_merge(vec, M, L, E, O);
        write_out(it, h, vec * 4 - h * D, O, M, L, E);
      }
    } else if (wave == 0) {
      for (int vec = lane; vec < NV; vec += kWave) {
        const int h = (vec * 4) / D;
        if (h >= it.nh) continue;
        float M, L, E;
        float4_t O;
        wave_merge(vec, M, L, E, O);
        const int64_t ph = it.pidx * GT + h;
        st16_device(p.part_o, (uint32_t)((ph * D + vec * 4 - h * D) * 4), as_uint4f(O));
        if (vec * 4 == h * D)
          st16_device(p.part_ml, (uint32_t)(ph * 16), as_uint4f(float4_t{M, L, E, 0.f}));
      }
    }
    if constexpr (DEFER) {
      if (merge_pend) {  // workgroup-uniform
        if (tid == 0) atomicExch(&p.arrive[sm_pend.unit], 0);
        __syncthreads();  // the merge buffers are read above
        merge_unit(sm_pend);
      }
    } else {
      if (!it.direct && arrive_now(it)) merge_unit(it);  // workgroup-uniform
    }
    __syncthreads();  // the merge buffers are reused by the next item
    if constexpr (DEFER) {
      // Every read of the previous sm_pend is above the barrier; thread 0
      // itself reads the new one next, the other threads after later barriers.
      has_pend = !it.direct;
      if (has_pend && tid == 0) sm_pend = it;
    }
    return next_ticket;
  };

  // Sequence bb has no tokens: o = 0 and lse = -inf for all its query heads.
  auto zero_sequence = [&](int bb) {
    half_t* orow = p.o + (int64_t)bb * p.Hq * D;
    for (int i = tid; i < p.Hq * (D / 8); i += kThreads) st16(orow + 8 * i, uint4_t{0, 0, 0, 0});
    if (p.lse)
      for (int h = tid; h < p.Hq; h += kThreads) p.lse[(int64_t)bb * p.Hq + h] = AKT_NEG_INF;
  };

  // ---- drivers ---------------------------------------------------------------
  if constexpr (PERSIST) {
    int n_items;
    // LDS starts with whatever the CU's previous workgroup left: sm_tick
    // must read 0 before any wave can compare it (barriers below).
    if (tid == 0) sm_tick = 0;
    if constexpr (TABLE) {
      // Chunk prefix over sequences (block-wide exclusive scan), once.
      int carry = 0;
      for (int base = 0; base < p.B; base += kThreads) {
        const int bb = base + tid;
        int n = 0, len = 0, ps = 0;
        if (bb < p.B) {
          ps = p.indptr[bb];
          len = paged_len(p.indptr, p.last_len, bb, p.page_size);
          n = (len + p.chunk - 1) / p.chunk;
        }
        int incl = n;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int t = __shfl_up(incl, off, 64);
          if (lane >= off) incl += t;
        }
        if (lane == 63) sm_wtot[wave] = incl;
        __syncthreads();
        int before = carry, total = carry;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          before += (w < wave) ? sm_wtot[w] : 0;
          total += sm_wtot[w];
        }
        if (bb < p.B) {
          sm_cs[bb] = before + incl - n;
          sm_len[bb] = len;
          sm_ps[bb] = ps;
        }
        carry = total;
        __syncthreads();
      }
      if (tid == 0) sm_cs[p.B] = carry;
      __syncthreads();
      n_items = sm_cs[p.B] * Y;
      // Sequences without tokens have no items: their rows are written here.
      for (int bb = blockIdx.x; bb < p.B; bb += gridDim.x)
        if (sm_len[bb] == 0) zero_sequence(bb);
    } else {
      n_items = p.B * ((p.S + p.chunk - 1) / p.chunk) * Y;
      __syncthreads();  // sm_tick
    }
    // The item whose first groups the current item's last iterations
    // prefetch.  Past the last item it is the current one with an empty
    // token range: every lane then reads the unit's q row (an L2 hit) instead
    // of re-reading K/V that left the cache long ago.
    auto resolve_next = [&](int inext, int icur) -> Item {
      if (inext < n_items) return resolve_persistent(inext);
      Item w = resolve_persistent(icur);
      w.t1 = w.t0;
      return w;
    };
    // Dynamic schedule: workgroup w starts with item w, then takes tickets
    // from counters[0] (item gridDim.x + ticket); the last workgroup to exit
    // resets both counters to zero for the next launch.
    // - Long items (NEAR, GPW >= 6): the ticket thread 0 takes after group
    //   kAtomicK names the next item.  Thread 0 publishes it in LDS after
    //   group kPublishK (with the item count, in sm_tick) and every
    //   wave sets the next item up after group kTicketK, in time for the
    //   prefetch of its first groups.  When the tickets run out a workgroup
    //   has at most the rest of its current item and one more left, so the
    //   last workgroups to finish trail the mean by about one item.
    // - Short items: the ticket names the item after next (items w and
    //   w + gridDim.x start the walk), read back at the workgroup merge, so
    //   the atomic's latency stays hidden even in a two-group item.
    constexpr bool NEAR = GPW >= 6 && PD == 2;
    constexpr int kTicketK = GPW - 4;                     // next item set up
    constexpr int kPublishK = kTicketK - 1;               // ticket in LDS
    constexpr int kAtomicK = kPublishK >= 3 ? kPublishK - 2 : 0;  // ticket taken
    int i = blockIdx.x;
    int nxt = i + (int)gridDim.x;
    int ticket_raw = 0;  // thread 0: counters[0] before its increment
    int seq = 0;         // items this workgroup has begun
    if (i < n_items) {  // workgroup-uniform; the grid is sized from an upper bound
    Item nx;
    IssueCtx cc, nc;
    half8_t qn[KS];
    it = resolve_persistent(i);
    make_uniform(it);
    setup(it, cc, qf);
    if constexpr (!NEAR) {
      nx = resolve_next(nxt, i);
      make_uniform(nx);
      setup(nx, nc, qn);
    }
    Buf bufs[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) issue(cc, cc.g_begin + wave + kWaves * j, bufs[j]);
    for (;;) {
      // The returned value is first used two groups later (NEAR) or at the
      // item's end: using it at once would make the wave wait for the loads
      // in flight.
      if constexpr (!NEAR) {
        if (tid == 0) ticket_raw = atomicAdd(&p.counters[0], 1);
      }
      begin_item();
      ++seq;
      // Groups k of this item; the prefetch PD groups ahead crosses into the
      // next item for the last PD (k + PD >= GPW is a compile-time condition).
#pragma unroll
      for (int k = 0; k < GPW; ++k) {
        consume(bufs[k % PD]);
        if constexpr (NEAR) {
          if (k == kAtomicK && tid == 0) ticket_raw = atomicAdd(&p.counters[0], 1);
          if (k == kPublishK && tid == 0) {
            // Waiting for the ticket waits for the loads issued before the
            // atomic (groups up to kAtomicK + 1, all consumed) and no others.
            lds_store_u64(&sm_tick, (uint32_t)((int)gridDim.x + ticket_raw) |
                                        ((unsigned long long)(uint32_t)seq << 32));
          }
          if (k == kTicketK) {
            // Thread 0 wrote this item's ticket after group kPublishK; a
            // wave this far ahead of wave 0 waits for it.  The previous item's
            // reads of sm_next all precede the workgroup merge's barrier,
            // which precedes thread 0's next write.
            unsigned long long tk = lds_load_u64(&sm_tick);
            while ((int)(tk >> 32) != seq) {
              __builtin_amdgcn_s_sleep(1);
              tk = lds_load_u64(&sm_tick);
            }
            nxt = uniform((int)(uint32_t)tk);
            nx = resolve_next(nxt, i);
            make_uniform(nx);
            setup(nx, nc, qn);
          }
        }
        if constexpr (DEFER) {
          if (k == PD && has_pend && tid == 0) {
            // Group PD's loads, the first issued in this item, were issued
            // after the pending partial's stores (at the previous finish()),
            // and wave 0 has just waited for them: in-order completion makes
            // those stores complete too.  The empty asm consumes a word of
            // group PD and yields 0, so the count cannot be issued before
            // that wait.
            int zero = 0;
            asm volatile("" : "+s"(zero) : "v"(bufs[0].k[0][0]));
            arr = atomicAdd(&p.arrive[sm_pend.unit + zero], 1);
          }
        }
        if (k + PD < GPW) issue(cc, cc.g_begin + wave + kWaves * (k + PD), bufs[k % PD]);
        else issue(nc, nc.g_begin + wave + kWaves * (k + PD - GPW), bufs[k % PD]);
      }
      if (tid == 0) {  // read back by finish() after its first barrier
        // (NEAR: a wave behind wave 0 may still have to read this item's
        // ticket from sm_next, so it is not rewritten here.)
        if constexpr (!NEAR) sm_next = 2 * (int)gridDim.x + ticket_raw;
        if constexpr (DEFER) sm_pflag = has_pend && arr == sm_pend.nch - 1;
      }
      const int ticket = finish();
      const int inext = nxt;
      if constexpr (!NEAR) nxt = ticket;
      if (inext >= n_items) break;  // the last prefetch read q rows (see resolve_next)
      i = inext;
      it = nx;
      cc = nc;
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s] = qn[s];
      if constexpr (!NEAR) {
        nx = resolve_next(nxt, i);
        make_uniform(nx);
        setup(nx, nc, qn);
      }
    }
    }  // i < n_items
    if constexpr (DEFER) {
      // The last item's partial has not been counted yet.
      if (has_pend && arrive_now(sm_pend)) merge_unit(sm_pend);  // workgroup-uniform
    }
    if (tid == 0) {
      if (atomicAdd(&p.counters[1], 1) == (int)gridDim.x - 1) {
        atomicExch(&p.counters[0], 0);
        atomicExch(&p.counters[1], 0);
      }
    }
  } else {
    if constexpr (MODE == kModePaged) {
      // Sequences without tokens have no chunk (grid.x >= B).
      if (blockIdx.y == 0 && (int)blockIdx.x < p.B &&
          paged_len(p.indptr, p.last_len, blockIdx.x, p.page_size) == 0)
        zero_sequence(blockIdx.x);
    }
    it = resolve_block();
    if (it.b < 0) return;  // workgroup-uniform
    make_uniform(it);
    IssueCtx cc;
    setup(it, cc, qf);
    begin_item();
    const int g_end = (it.t1 + 15) >> 4;
    if constexpr (GPW > 0) {
      Buf bufs[2];
      const int gw = cc.g_begin + wave;
      issue(cc, gw, bufs[0]);
#pragma unroll
      for (int k = 0; k < GPW; ++k) {
        if (k + 1 < GPW) issue(cc, gw + kWaves * (k + 1), bufs[(k + 1) & 1]);
        consume(bufs[k & 1]);
      }
    } else {
      // Dynamic group count (sparse units): ping-pong over two buffers.  The
      // last prefetch re-reads the current group (an L2 hit) so that every
      // iteration issues the same loads.
      int g = cc.g_begin + wave;
      if (g < g_end) {
        Buf A, B;
        issue(cc, g, A);
        for (;;) {
          int gn = g + kWaves;
          issue(cc, gn < g_end ? gn : g, B);
          consume(A);
          if (gn >= g_end) break;
          g = gn;
          gn = g + kWaves;
          issue(cc, gn < g_end ? gn : g, A);
          consume(B);
          if (gn >= g_end) break;
          g = gn;
        }
      }
    }
    finish();
  }
}

// ---------------------------------------------------------------------------
// Rows of an empty dense cache: o = 0, lse = -inf.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void empty_rows_kernel(half_t* o, float* lse, int64_t rows,
                                                              int D) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < rows * (D / 8)) st16(o + 8 * i, uint4_t{0, 0, 0, 0});
  if (lse && i < rows) lse[i] = AKT_NEG_INF;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

int pick_gt(int G, int D) {
  const int gmax = (D == 256) ? 8 : 16;
  int gt = 1;
  while (gt < G && gt < gmax) gt <<= 1;
  return gt;
}

// Launches one split-kernel instance.  Persistent instances get a grid of
// min(items, resident workgroups); `grid` carries the item upper bound in x.
template <int D, int GT, int MODE, bool ALIGNED, bool MAGIC, int GPW, bool PERSIST>
int launch_split(const SplitParams& p, dim3 grid, hipStream_t st) {
  auto kernel = split_kernel<D, GT, MODE, ALIGNED, MAGIC, GPW, PERSIST>;
  if (PERSIST) {
    const int64_t items = (int64_t)grid.x * grid.y;
    const int cap = resident_blocks(kernel, kThreads);
    if (cap <= 0) return set_error(AKT_ERR_HIP, "occupancy query failed");
    grid = dim3((unsigned)(items < cap ? items : cap), 1);
  }
  KernelTimer timer;
  timer.launch(kernel, grid, dim3(kThreads), 0, st, p);
  return check_launch("split_kernel");
}

template <int D, int GT, int MODE, bool ALIGNED, bool MAGIC>
int launch_t(const SplitParams& p, dim3 grid, hipStream_t st) {
  constexpr bool SPARSE = (MODE == kModeSparseDense || MODE == kModeSparsePaged);
  if constexpr (SPARSE) {
    return launch_split<D, GT, MODE, ALIGNED, MAGIC, 0, false>(p, grid, st);
  } else if constexpr (MODE == kModePaged && !ALIGNED) {
    // Pages that do not hold whole 16-token groups: 256-token chunks only.
    if (p.B <= kMaxTableB) return launch_split<D, GT, MODE, false, MAGIC, 4, true>(p, grid, st);
    return launch_split<D, GT, MODE, false, MAGIC, 4, false>(p, grid, st);
  } else {
    // A chunk of `chunk` tokens is chunk / 64 16-token groups per wave.
    if constexpr (MODE == kModePaged) {
      if (p.B > kMaxTableB) return launch_split<D, GT, MODE, ALIGNED, MAGIC, 4, false>(p, grid, st);
    }
    if (p.chunk == 128) return launch_split<D, GT, MODE, ALIGNED, MAGIC, 2, true>(p, grid, st);
    if (p.chunk == 256) return launch_split<D, GT, MODE, ALIGNED, MAGIC, 4, true>(p, grid, st);
    if (p.chunk == 640) return launch_split<D, GT, MODE, ALIGNED, MAGIC, 10, true>(p, grid, st);
    return launch_split<D, GT, MODE, ALIGNED, MAGIC, 8, true>(p, grid, st);
  }
}

template <int D, int MODE, bool ALIGNED, bool MAGIC>
int launch_gt(int gt, const SplitParams& p, dim3 grid, hipStream_t st) {
  if constexpr (MODE == kModeSparseDense || MODE == kModeSparsePaged) {
    return launch_t<D, 1, MODE, ALIGNED, MAGIC>(p, grid, st);
  } else {
    switch (gt) {
      case 1: return launch_t<D, 1, MODE, ALIGNED, MAGIC>(p, grid, st);
      case 2: return launch_t<D, 2, MODE, ALIGNED, MAGIC>(p, grid, st);
      case 4: return launch_t<D, 4, MODE, ALIGNED, MAGIC>(p, grid, st);
      case 8: return launch_t<D, 8, MODE, ALIGNED, MAGIC>(p, grid, st);
      case 16:
        if constexpr (D != 256) return launch_t<D, 16, MODE, ALIGNED, MAGIC>(p, grid, st);
        break;
    }
    return set_error(AKT_ERR_UNSUPPORTED, "no decode kernel for %d heads per unit", gt);
  }
}

template <int MODE, bool ALIGNED, bool MAGIC>
int launch_d(int D, int gt, const SplitParams& p, dim3 grid, hipStream_t st) {
  switch (D) {
    case 64: return launch_gt<64, MODE, ALIGNED, MAGIC>(gt, p, grid, st);
    case 128: return launch_gt<128, MODE, ALIGNED, MAGIC>(gt, p, grid, st);
    case 256: return launch_gt<256, MODE, ALIGNED, MAGIC>(gt, p, grid, st);
  }
  return set_error(AKT_ERR_UNSUPPORTED, "head_dim %d not supported (64, 128, 256)", D);
}

// Workspace layout of a split launch: the counter header, the arrival
// counters, then the partial outputs [parts, GT, D] and their (m, l, e, pad)
// rows [parts, GT, 4], all fp32.  Arrival counters must be zero when a launch
// starts and every launch leaves its own at zero, but a workspace is shared by
// calls of different shapes, so partials of one call must never land where
// another call looks for counters: the first kArriveSlots counters sit in a
// fixed area that partials never use, and a call with more units than that
// also zero-fills its extra counters (which may hold an earlier call's
// partials) before the split kernel runs.  Launches without partials (every
// unit a single chunk) need no counters.  Partials are addressed with 32-bit
// byte offsets, so each array must stay below 2 GiB.
constexpr int64_t kArriveSlots = 32768;
static_assert(kCounterBytes + kArriveSlots * 4 == AKT_WORKSPACE_ZERO_BYTES,
              "the public zero-prefix size matches the workspace layout");

struct WsLayout {
  size_t arrive, extra_bytes, part_o, part_ml, total;
  bool fits;
};

WsLayout ws_layout(int64_t units, int64_t parts, int gt, int64_t D) {
  WsLayout w = {};
  w.fits = true;
  w.arrive = kCounterBytes;
  if (parts == 0) {
    w.part_o = w.part_ml = w.total = kCounterBytes;
    return w;
  }
  const int64_t slots = units > kArriveSlots ? units : kArriveSlots;
  const int64_t po = parts * gt * D * 4, pml = parts * gt * 16;
  w.extra_bytes = (size_t)(slots - kArriveSlots) * 4;
  w.part_o = w.arrive + (size_t)round_up(slots * 4, 256);
  w.part_ml = w.part_o + (size_t)round_up(po, 256);
  w.total = w.part_ml + (size_t)pml;
  w.fits = po < kMaxPartialBytes && pml < kMaxPartialBytes;
  return w;
}

// Points the kernel's counters and partials into `ws`.
void bind_workspace(SplitParams& p, void* ws, const WsLayout& w) {
  char* c = (char*)ws;
  p.counters = (int*)c;
  p.arrive = (int*)(c + w.arrive);
  p.part_o = (float*)(c + w.part_o);
  p.part_ml = (float*)(c + w.part_ml);
}

__global__ __launch_bounds__(kThreads) void zero_words_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Zero-fills the arrival counters past the fixed area (see ws_layout).
int clear_extra_arrivals(const SplitParams& p, const WsLayout& w, hipStream_t st) {
  if (w.extra_bytes == 0) return AKT_OK;
  const int64_t n = (int64_t)(w.extra_bytes / 4);
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                     st, p.arrive + kArriveSlots, n);
  return check_launch("zero_words_kernel");
}

int check_workspace(const WsLayout& w, const void* ws, size_t ws_bytes) {
  if (!w.fits)
    return set_error(AKT_ERR_UNSUPPORTED, "split-KV partials exceed 2 GiB; use longer chunks");
  if (!ws || ws_bytes < w.total)
    return set_error(AKT_ERR_WORKSPACE, "workspace of %zu bytes required", w.total);
  return AKT_OK;
}

// Workgroups of the decode kernels resident at once on MI355X: two per CU
// (VGPR-bound) on 256 CUs.
constexpr int64_t kResidentWorkgroups = 512;

// Automatic chunk length for dense / paged caches.  An item carries a fixed
// cost (the workgroup merge, a partial, its share of the combine) that small
// chunks do not amortise, while the last items set the launch's tail:
// - the smallest of 128, 256 and 512 that cuts the launch into at most ~256
//   items (in practice 512 unless the launch is tiny): measured on MI355X,
//   512 beats 128 and 256 for config 2 (dense, 256 items) and config 3;
// - 640 when even a lower bound on its item count (total tokens / 640 per
//   unit) leaves each of the ~512 resident workgroups (two per CU) at least
//   2.75 items.  Config 3 (paged, 1569 items), nine in-process pairs on
//   three MI355X boxes: 92.3-94.4 us against 94.0-96.7 at 512 (mean -1.2 us);
//   768-token chunks (2.6 items per workgroup) took 97-98 us.
int64_t auto_chunk(int64_t total_tokens, int64_t units) {
  if ((total_tokens / 640) * units * 4 >= kResidentWorkgroups * 11) return 640;
  const int64_t want = ceil_div(total_tokens * units, 256);
  int64_t c = 128;
  while (c < want && c < 512) c <<= 1;
  return c;
}

bool chunk_ok(int64_t c) { return c == 0 || c == 128 || c == 256 || c == 512 || c == 640; }

// Chunk length of a paged launch: pages that do not hold whole 16-token
// groups and batches past the LDS chunk table use 256-token chunks.
int64_t paged_chunk(int64_t chunk_tokens, int64_t total_pages, int64_t page_size, int64_t Y,
                    int64_t batch) {
  if (page_size % 16 != 0 || batch > kMaxTableB) return 256;
  return chunk_tokens > 0 ? chunk_tokens : auto_chunk(total_pages * page_size, Y);
}

// Automatic split count of sparse rows: as many splits per row as fit one
// round of resident workgroups, at most kMaxAutoSplits and at most one per 64
// index slots.  A sparse workgroup is a chain of dependent round trips (nnz,
// page table, indices, page ids, rows) whatever its token count, so a second
// round of workgroups costs a whole second chain, and a split of a few
// groups pays the chain for little streaming.  Measured on MI355X (split
// kernel, settled, rotated inputs):
//   config 4a (32 rows):  32 splits 16.4 us, 16 splits 9.8 us, 12 / 8 / 4
//                         splits 9.1 / 9.2 / 9.1 us, 2 splits 11.4 us;
//   config 4b (96 rows):  11 splits 23.8 us, 8 splits 29.1 us, 5 splits
//                         18.7 us, 4 splits 19.3 us, 2 splits 20.4 us.
constexpr int64_t kMaxAutoSplits = 8;
int64_t auto_splits(int64_t rows, int64_t l_max) {
  int64_t s = kResidentWorkgroups / (rows > 0 ? rows : 1);
  if (s > kMaxAutoSplits) s = kMaxAutoSplits;
  const int64_t cap = ceil_div(l_max > 0 ? l_max : 1, 64);
  if (s > cap) s = cap;
  return s < 1 ? 1 : s;
}

bool head_dim_ok(int64_t D) { return D == 64 || D == 128 || D == 256; }

int check_common(int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
  AKT_CHECK(B >= 0 && Hq > 0 && Hkv > 0, "batch/head counts must be positive");
  AKT_CHECK(Hq % Hkv == 0, "num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)",
            (long long)Hq, (long long)Hkv);
  if (!head_dim_ok(D))
    return set_error(AKT_ERR_UNSUPPORTED, "head_dim %lld not supported (64, 128, 256)", (long long)D);
  return AKT_OK;
}

}  // namespace
}  // namespace akt

using namespace akt;

// ----------------------------- dense decode --------------------------------
extern "C" size_t akt_decode_workspace_size(int64_t batch, int64_t num_q_heads,
                                            int64_t num_kv_heads, int64_t seq_len,
                                            int64_t head_dim, int64_t chunk_tokens) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || !head_dim_ok(head_dim)) return 0;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, (int)head_dim);
  const int64_t Y = num_kv_heads * ceil_div(G, gt);
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(seq_len * batch, Y);
  const int64_t nch = ceil_div(seq_len, chunk);
  return ws_layout(batch * Y, nch > 1 ? batch * Y * nch : 0, gt, head_dim).total;
}

extern "C" int akt_decode_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                              int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                              int64_t seq_len, int64_t head_dim, const int64_t q_stride[4],
                              const int64_t k_stride[4], const int64_t v_stride[4],
                              float softmax_scale, int64_t chunk_tokens, void* workspace,
                              size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common(batch, num_q_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  AKT_CHECK(seq_len >= 0 && seq_len < (1ll << 31), "seq_len out of range");
  AKT_CHECK(q_stride[3] == 1 && k_stride[3] == 1 && v_stride[3] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 3) && rows_aligned16(k, k_stride, 3) &&
                rows_aligned16(v, v_stride, 3) && aligned16(o),
            "tensors must have 16-byte aligned rows");
  AKT_CHECK(chunk_ok(chunk_tokens), "chunk_tokens must be 0 (automatic), 128, 256, 512 or 640");
  if (batch == 0) return AKT_OK;
  const int D = (int)head_dim;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, D);
  const int n_hg = (int)ceil_div(G, gt);
  const int64_t Y = num_kv_heads * n_hg;
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(seq_len * batch, Y);
  const int64_t nch = ceil_div(seq_len, chunk);
  const WsLayout wl = ws_layout(batch * Y, nch > 1 ? batch * Y * nch : 0, gt, D);
  rc = check_workspace(wl, workspace, workspace_bytes);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (nch == 0) {  // empty cache: every row is o = 0, lse = -inf
    const int64_t rows = batch * num_q_heads;
    hipLaunchKernelGGL(empty_rows_kernel, dim3((unsigned)ceil_div(rows * (D / 8), kThreads)),
                       dim3(kThreads), 0, st, (half_t*)o, lse, rows, D);
    return check_launch("empty_rows_kernel");
  }

  SplitParams p = {};
  p.q = (const half_t*)q;
  p.kbase = (const half_t*)k;
  p.vbase = (const half_t*)v;
  p.o = (half_t*)o;
  p.lse = lse;
  bind_workspace(p, workspace, wl);
  p.q_sb = q_stride[0];
  p.q_sh = q_stride[1];
  p.k_sa = k_stride[2]; p.k_sb = 0; p.k_batch = k_stride[0]; p.k_head = k_stride[1];
  p.v_sa = v_stride[2]; p.v_sb = 0; p.v_batch = v_stride[0]; p.v_head = v_stride[1];
  p.B = (int)batch; p.Hq = (int)num_q_heads; p.Hkv = (int)num_kv_heads; p.G = G;
  p.S = (int)seq_len;
  p.n_hg = n_hg;
  p.chunk = (int)chunk;
  p.qk_scale = softmax_scale * kLog2e;
  rc = clear_extra_arrivals(p, wl, st);
  if (rc) return rc;
  return launch_d<kModeDense, false, false>(D, gt, p, dim3((unsigned)(batch * nch), (unsigned)Y), st);
}

// ----------------------------- paged decode --------------------------------
static int64_t paged_grid_x(int64_t total_pages, int64_t page_size, int64_t chunk, int64_t batch) {
  return ceil_div(total_pages * page_size, chunk) + batch;
}

// The stream-K kernel (paged_stream.hip) serves the automatic chunk length
// whenever it can; explicit chunk lengths keep the chunked split kernel.
static bool use_stream(int64_t chunk_tokens, int64_t batch, int64_t page_size,
                       int64_t total_pages, int64_t Y) {
  return chunk_tokens == 0 && paged_stream_eligible(batch, page_size, total_pages, Y);
}

static WsLayout paged_layout(int64_t batch, int64_t Y, int gt, int64_t D, int64_t page_size,
                             int64_t total_pages, int64_t chunk_tokens) {
  if (use_stream(chunk_tokens, batch, page_size, total_pages, Y))
    return ws_layout(batch * Y, paged_stream_wave_cap((int)D, gt) + batch * Y, gt, D);
  const int64_t chunk = paged_chunk(chunk_tokens, total_pages, page_size, Y, batch);
  return ws_layout(batch * Y, paged_grid_x(total_pages, page_size, chunk, batch) * Y, gt, D);
}

extern "C" size_t akt_decode_paged_workspace_size(int64_t batch, int64_t num_q_heads,
                                                  int64_t num_kv_heads, int64_t head_dim,
                                                  int64_t page_size, int64_t total_pages,
                                                  int64_t chunk_tokens) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || !head_dim_ok(head_dim) ||
      page_size <= 0)
    return 0;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, (int)head_dim);
  const int64_t Y = num_kv_heads * ceil_div(G, gt);
  return paged_layout(batch, Y, gt, head_dim, page_size, total_pages, chunk_tokens).total;
}

namespace akt {
int paged_decode_impl(const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
                      const int32_t* kv_page_indices, const int32_t* kv_last_page_len, void* o,
                      float* lse, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                      int64_t head_dim, int64_t page_size, int64_t total_pages,
                      int64_t num_pool_pages, const int64_t q_stride[4],
                      const int64_t kv_stride[5], float softmax_scale, int64_t chunk_tokens,
                      void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(batch, num_q_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  AKT_CHECK(page_size > 0 && page_size < (1 << 20), "page_size out of range");
  AKT_CHECK(total_pages >= 0 && num_pool_pages >= 0 && total_pages * page_size < (1ll << 31),
            "page counts out of range");
  AKT_CHECK(q_stride[3] == 1 && kv_stride[4] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 3) && rows_aligned16(kv_cache, kv_stride, 4) && aligned16(o),
            "tensors must have 16-byte aligned rows");
  AKT_CHECK(chunk_ok(chunk_tokens), "chunk_tokens must be 0 (automatic), 128, 256, 512 or 640");
  // A group's 16 rows are addressed with 32-bit byte offsets from its first.
  AKT_CHECK(kv_stride[3] >= 0 && kv_stride[3] < (1 << 26), "kv_cache row stride out of range");
  if (batch == 0) return AKT_OK;
  const int D = (int)head_dim;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, D);
  const int n_hg = (int)ceil_div(G, gt);
  const int64_t Y = num_kv_heads * n_hg;
  const WsLayout wl = paged_layout(batch, Y, gt, D, page_size, total_pages, chunk_tokens);
  rc = check_workspace(wl, workspace, workspace_bytes);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (use_stream(chunk_tokens, batch, page_size, total_pages, Y)) {
    StreamParams sp = {};
    sp.q = (const half_t*)q;
    sp.kbase = (const half_t*)kv_cache;
    sp.vbase = (const half_t*)kv_cache + kv_stride[1];
    sp.indptr = kv_page_indptr;
    sp.indices = kv_page_indices;
    sp.last_len = kv_last_page_len;
    sp.o = (half_t*)o;
    sp.lse = lse;
    char* c = (char*)workspace;
    sp.arrive = (int*)(c + wl.arrive);
    sp.part_o = (float*)(c + wl.part_o);
    sp.part_ml = (float*)(c + wl.part_ml);
    sp.q_sb = q_stride[0];
    sp.q_sh = q_stride[1];
    sp.k_sa = kv_stride[0]; sp.k_head = kv_stride[2]; sp.k_sb = (int)kv_stride[3];
    sp.v_sa = kv_stride[0]; sp.v_head = kv_stride[2]; sp.v_sb = (int)kv_stride[3];
    sp.B = (int)batch; sp.Hq = (int)num_q_heads; sp.G = G; sp.Y = (int)Y; sp.n_hg = n_hg;
    sp.page_size = (int)page_size;
    sp.gpp = (int)(page_size / 16);
    sp.total_pages = (int)total_pages;
    sp.TG = (int)(total_pages * sp.gpp);
    sp.N = (int)(Y * sp.TG);
    sp.num_pool_pages = (int)(num_pool_pages < (1ll << 31) ? num_pool_pages : (1ll << 31) - 1);
    sp.qk_scale = softmax_scale * kLog2e;
    SplitParams cp = {};
    cp.arrive = sp.arrive;
    rc = clear_extra_arrivals(cp, wl, st);
    if (rc) return rc;
    return paged_stream_launch(sp, D, gt, st);
  }
  const int64_t chunk = paged_chunk(chunk_tokens, total_pages, page_size, Y, batch);
  const int64_t gx = paged_grid_x(total_pages, page_size, chunk, batch);

  SplitParams p = {};
  p.q = (const half_t*)q;
  p.kbase = (const half_t*)kv_cache;
  p.vbase = (const half_t*)kv_cache + kv_stride[1];
  p.indptr = kv_page_indptr;
  p.indices = kv_page_indices;
  p.last_len = kv_last_page_len;
  p.o = (half_t*)o;
  p.lse = lse;
  bind_workspace(p, workspace, wl);
  p.q_sb = q_stride[0];
  p.q_sh = q_stride[1];
  p.k_sa = kv_stride[0]; p.k_sb = kv_stride[3]; p.k_head = kv_stride[2];
  p.v_sa = kv_stride[0]; p.v_sb = kv_stride[3]; p.v_head = kv_stride[2];
  p.B = (int)batch; p.Hq = (int)num_q_heads; p.Hkv = (int)num_kv_heads; p.G = G;
  p.page_size = (int)page_size;
  p.num_pool_pages = (int)(num_pool_pages < (1ll << 31) ? num_pool_pages : (1ll << 31) - 1);
  p.n_hg = n_hg;
  p.chunk = (int)chunk;
  p.qk_scale = softmax_scale * kLog2e;
  // grid.x >= batch: the non-persistent form writes empty sequences' rows from
  // workgroups blockIdx.x < batch.
  const dim3 grid((unsigned)gx, (unsigned)Y);
  rc = clear_extra_arrivals(p, wl, st);
  if (rc) return rc;
  if (page_size % 16 == 0) return launch_d<kModePaged, true, false>(D, gt, p, grid, st);
  return launch_d<kModePaged, false, false>(D, gt, p, grid, st);
}
}  // namespace akt

extern "C" int akt_decode_paged_fwd(const void* q, const void* kv_cache,
                                    const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                    const int32_t* kv_last_page_len, void* o, float* lse,
                                    int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                    int64_t head_dim, int64_t page_size, int64_t total_pages,
                                    int64_t num_pool_pages, const int64_t q_stride[4],
                                    const int64_t kv_stride[5], float softmax_scale,
                                    int64_t chunk_tokens, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  clear_error();
  return paged_decode_impl(q, kv_cache, kv_page_indptr, kv_page_indices, kv_last_page_len, o, lse,
                           batch, num_q_heads, num_kv_heads, head_dim, page_size, total_pages,
                           num_pool_pages, q_stride, kv_stride, softmax_scale, chunk_tokens,
                           workspace, workspace_bytes, stream);
}

// ----------------------------- sparse decode -------------------------------
extern "C" size_t akt_sparse_decode_workspace_size(int64_t batch, int64_t num_q_heads,
                                                   int64_t head_dim, int64_t l_max,
                                                   int64_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || !head_dim_ok(head_dim)) return 0;
  const int64_t rows = batch * num_q_heads;
  const int64_t ns = num_splits > 0 ? num_splits : auto_splits(rows, l_max);
  return ws_layout(rows, ns > 1 ? rows * ns : 0, 1, head_dim).total;
}

namespace {

int sparse_common(SplitParams& p, const void* q, const int32_t* sparse_ind,
                  const int32_t* sparse_nnz, const int64_t* csr_ptr, void* o, float* lse,
                  int64_t batch,
                  int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t l_max,
                  const int64_t q_stride[4], const int64_t ind_stride[2],
                  const int64_t nnz_stride[2], int64_t num_splits, void* workspace,
                  size_t workspace_bytes, int64_t& ns_out, WsLayout& wl_out) {
  int rc = check_common(batch, num_q_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  AKT_CHECK(l_max >= 0 && l_max < (1ll << 31), "l_max out of range");
  AKT_CHECK(q_stride[3] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 2) && aligned16(o), "tensors must have 16-byte aligned rows");
  AKT_CHECK(num_splits >= 0, "num_splits must be >= 0");
  ns_out = 0;
  if (batch == 0) return AKT_OK;  // nothing to compute: no workspace needed
  const int64_t rows = batch * num_q_heads;
  const int64_t ns = num_splits > 0 ? num_splits : auto_splits(rows, l_max);
  const WsLayout wl = ws_layout(rows, ns > 1 ? rows * ns : 0, 1, head_dim);
  rc = check_workspace(wl, workspace, workspace_bytes);
  if (rc) return rc;
  wl_out = wl;
  p.q = (const half_t*)q;
  AKT_CHECK(csr_ptr || (sparse_nnz && (sparse_ind || l_max == 0) && ind_stride && nnz_stride),
            "kept-index pointers and strides are required");
  AKT_CHECK(!csr_ptr || sparse_ind,
            "CSR kept indices are required (a valid pointer even when every row is empty)");
  p.sparse_ind = sparse_ind;
  p.sparse_nnz = sparse_nnz;
  p.csr_ptr = csr_ptr;
  p.o = (half_t*)o;
  p.lse = lse;
  bind_workspace(p, workspace, wl);
  p.q_sb = q_stride[0];
  p.q_sh = q_stride[1];
  if (!csr_ptr) {
    p.ind_sb = ind_stride[0];
    p.ind_sh = ind_stride[1];
    p.nnz_sb = nnz_stride[0];
    p.nnz_sh = nnz_stride[1];
  }
  p.B = (int)batch; p.Hq = (int)num_q_heads; p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.l_max = (int)l_max;
  p.n_split = (int)ns;
  ns_out = ns;
  return AKT_OK;
}

}  // namespace

static int sparse_dense_impl(const void* q, const void* k, const void* v,
                             const int32_t* sparse_ind, const int32_t* sparse_nnz,
                             const int64_t* csr_ptr, void* o, float* lse, int64_t batch,
                             int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                             int64_t head_dim, int64_t l_max, const int64_t q_stride[4],
                             const int64_t k_stride[4], const int64_t v_stride[4],
                             const int64_t ind_stride[2], const int64_t nnz_stride[2],
                             float softmax_scale, int64_t num_splits, void* workspace,
                             size_t workspace_bytes, void* stream) {
  clear_error();
  SplitParams p = {};
  int64_t ns = 0;
  WsLayout wl = {};
  int rc = sparse_common(p, q, sparse_ind, sparse_nnz, csr_ptr, o, lse, batch, num_q_heads,
                         num_kv_heads, head_dim, l_max, q_stride, ind_stride, nnz_stride,
                         num_splits, workspace, workspace_bytes, ns, wl);
  if (rc) return rc;
  AKT_CHECK(seq_len >= 0 && seq_len < (1ll << 31), "seq_len out of range");
  AKT_CHECK(k_stride[3] == 1 && v_stride[3] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(k, k_stride, 3) && rows_aligned16(v, v_stride, 3),
            "tensors must have 16-byte aligned rows");
  if (batch == 0) return AKT_OK;
  p.kbase = (const half_t*)k;
  p.vbase = (const half_t*)v;
  p.k_sa = k_stride[2]; p.k_sb = 0; p.k_batch = k_stride[0]; p.k_head = k_stride[1];
  p.v_sa = v_stride[2]; p.v_sb = 0; p.v_batch = v_stride[0]; p.v_head = v_stride[1];
  p.S = (int)seq_len;
  p.qk_scale = softmax_scale * kLog2e;
  const int64_t rows = batch * num_q_heads;
  rc = clear_extra_arrivals(p, wl, (hipStream_t)stream);
  if (rc) return rc;
  return launch_d<kModeSparseDense, false, false>((int)head_dim, 1, p,
                                                  dim3((unsigned)(rows * ns), 1),
                                                  (hipStream_t)stream);
}

extern "C" int akt_sparse_decode_fwd(const void* q, const void* k, const void* v,
                                     const int32_t* sparse_ind, const int32_t* sparse_nnz,
                                     void* o, float* lse, int64_t batch, int64_t num_q_heads,
                                     int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                     int64_t l_max, const int64_t q_stride[4],
                                     const int64_t k_stride[4], const int64_t v_stride[4],
                                     const int64_t ind_stride[2], const int64_t nnz_stride[2],
                                     float softmax_scale, int64_t num_splits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return sparse_dense_impl(q, k, v, sparse_ind, sparse_nnz, nullptr, o, lse, batch, num_q_heads,
                           num_kv_heads, seq_len, head_dim, l_max, q_stride, k_stride, v_stride,
                           ind_stride, nnz_stride, softmax_scale, num_splits, workspace,
                           workspace_bytes, stream);
}

extern "C" int akt_sparse_decode_csr_fwd(const void* q, const void* k, const void* v,
                                         const int32_t* inds, const int64_t* ptr, void* o,
                                         float* lse, int64_t batch, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                         int64_t max_nnz, const int64_t q_stride[4],
                                         const int64_t k_stride[4], const int64_t v_stride[4],
                                         float softmax_scale, int64_t num_splits,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!ptr) {
    clear_error();
    return set_error(AKT_ERR_INVALID_ARGUMENT, "CSR row pointer is required");
  }
  return sparse_dense_impl(q, k, v, inds, nullptr, ptr, o, lse, batch, num_q_heads, num_kv_heads,
                           seq_len, head_dim, max_nnz, q_stride, k_stride, v_stride, nullptr,
                           nullptr, softmax_scale, num_splits, workspace, workspace_bytes, stream);
}

static int sparse_paged_impl(bool magic, const void* q, const void* kv_cache,
                             const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                             const int32_t* sparse_ind, const int32_t* sparse_nnz,
                             const int64_t* csr_ptr,
                             const float* lsh_k, const float* lsh_l, void* o, float* lse,
                             int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                             int64_t head_dim, int64_t page_size, int64_t num_pool_pages,
                             int64_t l_max, const int64_t q_stride[4], const int64_t kv_stride[5],
                             const int64_t ind_stride[2], const int64_t nnz_stride[2],
                             float softmax_scale, int64_t num_splits, void* workspace,
                             size_t workspace_bytes, void* stream) {
  clear_error();
  SplitParams p = {};
  int64_t ns = 0;
  WsLayout wl = {};
  int rc = sparse_common(p, q, sparse_ind, sparse_nnz, csr_ptr, o, lse, batch, num_q_heads,
                         num_kv_heads, head_dim, l_max, q_stride, ind_stride, nnz_stride,
                         num_splits, workspace, workspace_bytes, ns, wl);
  if (rc) return rc;
  AKT_CHECK(page_size > 0 && page_size < (1 << 20), "page_size out of range");
  AKT_CHECK(num_pool_pages >= 0, "num_pool_pages out of range");
  AKT_CHECK(kv_stride[4] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(kv_cache, kv_stride, 4), "tensors must have 16-byte aligned rows");
  if (magic) AKT_CHECK(lsh_k && lsh_l, "MagicPIG K and L are required");
  if (batch == 0) return AKT_OK;
  p.kbase = (const half_t*)kv_cache;
  p.vbase = (const half_t*)kv_cache + kv_stride[1];
  p.indptr = kv_page_indptr;
  p.indices = kv_page_indices;
  p.k_sa = kv_stride[0]; p.k_sb = kv_stride[3]; p.k_head = kv_stride[2];
  p.v_sa = kv_stride[0]; p.v_sb = kv_stride[3]; p.v_head = kv_stride[2];
  p.page_size = (int)page_size;
  p.num_pool_pages = (int)(num_pool_pages < (1ll << 31) ? num_pool_pages : (1ll << 31) - 1);
  p.qk_scale = softmax_scale * kLog2e;
  p.inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
  p.lsh_k = lsh_k;
  p.lsh_l = lsh_l;
  const int64_t rows = batch * num_q_heads;
  const dim3 grid((unsigned)(rows * ns), 1);
  hipStream_t st = (hipStream_t)stream;
  rc = clear_extra_arrivals(p, wl, st);
  if (rc) return rc;
  if (magic) return launch_d<kModeSparsePaged, false, true>((int)head_dim, 1, p, grid, st);
  return launch_d<kModeSparsePaged, false, false>((int)head_dim, 1, p, grid, st);
}

extern "C" int akt_sparse_decode_paged_fwd(
    const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
    const int32_t* kv_page_indices, const int32_t* sparse_ind, const int32_t* sparse_nnz, void* o,
    float* lse, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t page_size, int64_t num_pool_pages, int64_t l_max, const int64_t q_stride[4],
    const int64_t kv_stride[5], const int64_t ind_stride[2], const int64_t nnz_stride[2],
    float softmax_scale, int64_t num_splits, void* workspace, size_t workspace_bytes,
    void* stream) {
  return sparse_paged_impl(false, q, kv_cache, kv_page_indptr, kv_page_indices, sparse_ind,
                           sparse_nnz, nullptr, nullptr, nullptr, o, lse, batch, num_q_heads, num_kv_heads,
                           head_dim, page_size, num_pool_pages, l_max, q_stride, kv_stride,
                           ind_stride, nnz_stride, softmax_scale, num_splits, workspace,
                           workspace_bytes, stream);
}

extern "C" int akt_magicpig_decode_paged_fwd(
    const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
    const int32_t* kv_page_indices, const int32_t* sparse_ind, const int32_t* sparse_nnz,
    const float* lsh_k, const float* lsh_l, void* o, float* lse, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
    int64_t num_pool_pages, int64_t l_max, const int64_t q_stride[4], const int64_t kv_stride[5],
    const int64_t ind_stride[2], const int64_t nnz_stride[2], int64_t num_splits, void* workspace,
    size_t workspace_bytes, void* stream) {
  return sparse_paged_impl(true, q, kv_cache, kv_page_indptr, kv_page_indices, sparse_ind,
                           sparse_nnz, nullptr, lsh_k, lsh_l, o, lse, batch, num_q_heads,
                           num_kv_heads, head_dim, page_size, num_pool_pages, l_max, q_stride,
                           kv_stride, ind_stride, nnz_stride, 1.0f / sqrtf((float)head_dim),
                           num_splits, workspace, workspace_bytes, stream);
}

extern "C" int akt_sparse_decode_paged_csr_fwd(
    const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
    const int32_t* kv_page_indices, const int32_t* inds, const int64_t* ptr, const float* lsh_k,
    const float* lsh_l, void* o, float* lse, int64_t batch, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pool_pages,
    int64_t max_nnz, const int64_t q_stride[4], const int64_t kv_stride[5], int64_t num_splits,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!ptr) {
    clear_error();
    return set_error(AKT_ERR_INVALID_ARGUMENT, "CSR row pointer is required");
  }
  const bool magic = lsh_k || lsh_l;
  return sparse_paged_impl(magic, q, kv_cache, kv_page_indptr, kv_page_indices, inds, nullptr, ptr,
                           lsh_k, lsh_l, o, lse, batch, num_q_heads, num_kv_heads, head_dim,
                           page_size, num_pool_pages, max_nnz, q_stride, kv_stride, nullptr,
                           nullptr, 1.0f / sqrtf((float)head_dim), num_splits, workspace,
                           workspace_bytes, stream);
}

// ----------------------------- no-allocation paged decode ------------------
// akt_decode_paged_fwd_noalloc keeps its split-KV workspace in this
// file-scope device array instead of caller memory: each GPU the library
// runs on holds its own copy, at its own address, until the process ends.
// In host code the name `scratch` is only a stand-in for the symbol; the
// device address comes from hipGetSymbolAddress (per device, with that device
// current) and only that address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[AKT_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device (guarded)

// Device address of `scratch` on the current device.  The first call on a
// device looks it up and zero-fills the workspace's counter area (the
// scheduling counters and the fixed arrival counters, which every launch
// leaves at zero again) with a fill kernel on `st`, ahead of the first launch
// that uses it.
int scratch_for_current_device(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(AKT_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(AKT_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    const int64_t n = (int64_t)((kCounterBytes + kArriveSlots * 4) / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                       st, (int*)ptr, n);
    const int rc = check_launch("zero_words_kernel");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return AKT_OK;
}
}  // namespace

extern "C" int akt_decode_paged_fwd_noalloc(
    const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
    const int32_t* kv_page_indices, const int32_t* kv_last_page_len, void* o, float* lse,
    int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
    int64_t total_pages, int64_t num_pool_pages, const int64_t q_stride[4],
    const int64_t kv_stride[5], float softmax_scale, int64_t chunk_tokens, void* stream) {
  clear_error();
  // Invalid arguments size to 0 here and are reported by paged_decode_impl.
  const size_t need = akt_decode_paged_workspace_size(batch, num_q_heads, num_kv_heads, head_dim,
                                                      page_size, total_pages, chunk_tokens);
  if (need > (size_t)AKT_NOALLOC_SCRATCH_BYTES)
    return set_error(AKT_ERR_INVALID_ARGUMENT,
                     "this call needs %zu bytes of split-KV workspace; the no-allocation entry "
                     "point holds %zu (use akt_decode_paged_fwd with a caller workspace)",
                     need, (size_t)AKT_NOALLOC_SCRATCH_BYTES);
  if (batch == 0) return paged_decode_impl(q, kv_cache, kv_page_indptr, kv_page_indices,
                                           kv_last_page_len, o, lse, batch, num_q_heads,
                                           num_kv_heads, head_dim, page_size, total_pages,
                                           num_pool_pages, q_stride, kv_stride, softmax_scale,
                                           chunk_tokens, nullptr, 0, stream);
  void* ws = nullptr;
  const int rc = scratch_for_current_device((hipStream_t)stream, &ws);
  if (rc) return rc;
  return paged_decode_impl(q, kv_cache, kv_page_indptr, kv_page_indices, kv_last_page_len, o, lse,
                           batch, num_q_heads, num_kv_heads, head_dim, page_size, total_pages,
                           num_pool_pages, q_stride, kv_stride, softmax_scale, chunk_tokens, ws,
                           (size_t)AKT_NOALLOC_SCRATCH_BYTES, stream);
}
