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
// (m, l, o) that split_combine_kernel merges with a log-sum-exp combine.
//
// Per 16-token group a wave computes the 16 x GT score block with four (D=128)
// v_mfma_f32_16x16x32_f16: A = K rows (token = lane & 15, each lane holds a
// contiguous D/4-element slice of its row), B = q^T (head = lane & 15).  The
// result lands as S^T: lane l holds head l & 15 for tokens 4*(l >> 4) + r.
// P.V runs on the VALU with v_dot2_f32_f16 over token pairs; V is loaded so
// that each 16-lane row holds the same four tokens its score registers cover,
// which makes the probability broadcast a within-row shuffle.
#include <math.h>

#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {

enum : int { kModeDense = 0, kModePaged = 1, kModeSparseDense = 2, kModeSparsePaged = 3 };

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
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
  const float* lsh_k;
  const float* lsh_l;
  half_t* o;      // [B, Hq, D] contiguous
  float* lse;     // [B, Hq] or null
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

// Wave-cooperative: first global chunk and chunk count of sequence b.
__device__ void chunk_span(const SplitParams& p, int b, int& cs_out, int& nch_out) {
  const int lane = threadIdx.x & 63;
  int acc = 0, mine = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int bb = base + lane;
    if (bb < p.B && bb <= b) {
      int len = paged_len(p.indptr, p.last_len, bb, p.page_size);
      int n = (len + p.chunk - 1) / p.chunk;
      if (bb < b) acc += n;
      else mine = n;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    acc += __shfl_xor(acc, off, 64);
    mine += __shfl_xor(mine, off, 64);
  }
  cs_out = acc;
  nch_out = mine;
}

// ---------------------------------------------------------------------------
// Split kernel.
// ---------------------------------------------------------------------------
template <int D, int GT, int MODE, bool ALIGNED, bool MAGIC>
__global__ __launch_bounds__(kThreads) void split_kernel(SplitParams p) {
  constexpr int KPL = D / 4;                 // K elements per lane per group
  constexpr int KS = D / 32;                 // MFMA k-steps (8 elements each)
  constexpr int VTOK = (D == 64) ? 2 : 4;    // V tokens per lane per group
  constexpr int VDIM = (D == 256) ? 16 : 8;  // V dims per lane
  constexpr int VLD = VDIM / 8;              // 16-byte loads per V token
  constexpr int NPAIR = VTOK / 2;
  constexpr bool SPARSE = (MODE == kModeSparseDense || MODE == kModeSparsePaged);
  constexpr bool PAGED_ADDR = (MODE == kModePaged || MODE == kModeSparsePaged);
  static_assert(!SPARSE || GT == 1, "sparse units hold one query head");

  __shared__ float sm_o[kWaves][GT][D];
  __shared__ float sm_m[kWaves][GT];
  __shared__ float sm_l[kWaves][GT];
  __shared__ float sm_e[kWaves][GT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int R = lane >> 4;
  const int c16 = lane & 15;

  // ---- resolve the work item -------------------------------------------
  int b = 0, kvh = 0, hq0 = 0, nh = 1, t0 = 0, t1 = 0, pstart = 0, np = 0;
  int64_t pidx = 0;
  bool direct = false;
  const int* ind_row = nullptr;
  if constexpr (MODE == kModeDense) {
    const int nch = (p.S + p.chunk - 1) / p.chunk;
    const int x = blockIdx.x;
    b = x / nch;
    const int c = x - b * nch;
    const int y = blockIdx.y;
    kvh = y / p.n_hg;
    const int hg = y - kvh * p.n_hg;
    hq0 = kvh * p.G + hg * GT;
    nh = min(GT, p.G - hg * GT);
    t0 = c * p.chunk;
    t1 = min(p.S, t0 + p.chunk);
    pidx = (int64_t)x * gridDim.y + y;
    direct = (nch == 1);
  } else if constexpr (MODE == kModePaged) {
    int c, nch, len;
    if (!locate_chunk(p, blockIdx.x, b, c, nch, len)) return;
    const int y = blockIdx.y;
    kvh = y / p.n_hg;
    const int hg = y - kvh * p.n_hg;
    hq0 = kvh * p.G + hg * GT;
    nh = min(GT, p.G - hg * GT);
    t0 = c * p.chunk;
    t1 = min(len, t0 + p.chunk);
    pidx = (int64_t)blockIdx.x * gridDim.y + y;
    direct = (nch == 1);
    pstart = p.indptr[b];
    np = p.indptr[b + 1] - pstart;
  } else {
    const int x = blockIdx.x;
    const int u = x / p.n_split;
    const int c = x - u * p.n_split;
    b = u / p.Hq;
    hq0 = u - b * p.Hq;
    kvh = hq0 / p.G;
    nh = 1;
    int n = p.sparse_nnz[(int64_t)b * p.nnz_sb + (int64_t)hq0 * p.nnz_sh];
    n = min(max(n, 0), p.l_max);
    // Split c covers [c*per, min(n, (c+1)*per)); per is a multiple of 64 so
    // every split starts on a 16-token group and splits never share a group.
    const int per = ((n + p.n_split - 1) / p.n_split + 63) & ~63;
    t0 = c * per;
    t1 = max(t0, min(n, t0 + per));
    pidx = x;
    direct = (p.n_split == 1);
    ind_row = p.sparse_ind + (int64_t)b * p.ind_sb + (int64_t)hq0 * p.ind_sh;
    if constexpr (MODE == kModeSparsePaged) {
      pstart = p.indptr[b];
      np = p.indptr[b + 1] - pstart;
    }
  }

  const int64_t k_unit = PAGED_ADDR ? (int64_t)kvh * p.k_head
                                    : (int64_t)b * p.k_batch + (int64_t)kvh * p.k_head;
  const int64_t v_unit = PAGED_ADDR ? (int64_t)kvh * p.v_head
                                    : (int64_t)b * p.v_batch + (int64_t)kvh * p.v_head;
  const half_t* __restrict__ kb = p.kbase + k_unit;
  const half_t* __restrict__ vb = p.vbase + v_unit;

  // ---- query fragment (B operand): head hq0 + c16, dims R*KPL + 8s + e --
  half8_t qf[KS];
  {
    const bool hv = c16 < nh;
    const half_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(hq0 + (hv ? c16 : 0)) * p.q_sh + R * KPL;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4_t v = ld16(qrow + 8 * s);
      if (!hv) v = uint4_t{0, 0, 0, 0};
      qf[s] = as_half8(v);
    }
  }

  // MagicPIG: |q|^2 for the unit's head (valid in lanes with c16 == 0).
  float q_norm = 0.f;
  float lsh_k = 0.f, lsh_l = 0.f;
  if constexpr (MAGIC) {
    float qs = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4_t u = as_uint4(qf[s]);
#pragma unroll
      for (int j = 0; j < 4; ++j) qs = dot2(u[j], u[j], qs);
    }
    q_norm = sqrtf(rows_sum(qs));
    lsh_k = p.lsh_k[(int64_t)b * p.Hq + hq0];
    lsh_l = p.lsh_l[(int64_t)b * p.Hq + hq0];
  }

  float m_run = AKT_NEG_INF;  // running max of head c16 (log2 units)
  // Partial normalisers over this lane's tokens: l_part sums the fp16-rounded
  // probabilities that multiply V (so O is normalised consistently), e_part
  // the fp32 probabilities (for the log-sum-exp output).
  float l_part = 0.f;
  float e_part = 0.f;
  float acc[GT][VDIM];
#pragma unroll
  for (int h = 0; h < GT; ++h)
#pragma unroll
    for (int d = 0; d < VDIM; ++d) acc[h][d] = 0.f;

  const uint32_t kOnes = 0x3c003c00u;  // half2(1, 1)
  const int g_begin = t0 >> 4;
  const int g_end = (t1 + 15) >> 4;

  for (int g = g_begin + wave; g < g_end; g += kWaves) {
    const int gpos = g << 4;

    // ---- K lane: row of token gpos + c16 --------------------------------
    const int pos_k = gpos + c16;
    int ra = 0, rb = 0, gpage = 0;
    bool kval = pos_k < t1;
    if constexpr (MODE == kModeDense) {
      ra = pos_k;
    } else if constexpr (MODE == kModePaged) {
      if constexpr (ALIGNED) {
        const int lp = uniform(gpos / p.page_size);
        const int page = p.indices[pstart + lp];
        const bool page_ok = page >= 0 && page < p.num_pool_pages;
        kval = kval && page_ok;
        gpage = page_ok ? page : 0;
        ra = page;
        rb = gpos - lp * p.page_size + c16;
      } else {
        if (kval) {
          const int lp = pos_k / p.page_size;
          const int page = p.indices[pstart + lp];
          kval = page >= 0 && page < p.num_pool_pages;
          ra = page;
          rb = pos_k - lp * p.page_size;
        }
      }
    } else if constexpr (MODE == kModeSparseDense) {
      if (kval) {
        const int t = ind_row[pos_k];
        kval = t >= 0 && t < p.S;
        ra = t;
      }
    } else {  // sparse paged
      if (kval) {
        const int t = ind_row[pos_k];
        const int lp = t >= 0 ? t / p.page_size : -1;
        kval = t >= 0 && lp < np;
        if (kval) {
          const int page = p.indices[pstart + lp];
          kval = page >= 0 && page < p.num_pool_pages;
          ra = page;
          rb = t - lp * p.page_size;
        }
      }
    }
    if (!kval) { ra = 0; rb = 0; }
    const uint64_t vmask = __ballot(kval);  // bit t (< 16): token gpos + t usable

    uint4_t kreg[KS];
    {
      const half_t* kr = kb + (int64_t)ra * p.k_sa + (int64_t)rb * p.k_sb + R * KPL;
#pragma unroll
      for (int s = 0; s < KS; ++s) kreg[s] = kval ? ld16(kr + 8 * s) : uint4_t{0, 0, 0, 0};
    }

    // ---- V lane: tokens of this row ------------------------------------
    uint4_t vreg[VTOK][VLD];
#pragma unroll
    for (int i = 0; i < VTOK; ++i) {
      const int tt = (D == 64) ? (4 * R + 2 * (c16 >> 3) + i) : (4 * R + i);
      const bool vv = (vmask >> tt) & 1;
      int va, vbb;
      if constexpr (MODE == kModeDense) {
        va = gpos + tt;
        vbb = 0;
      } else if constexpr (MODE == kModePaged && ALIGNED) {
        va = gpage;  // the page is uniform over the group
        vbb = gpos - (gpos / p.page_size) * p.page_size + tt;
      } else {
        va = __shfl(ra, tt, 64);
        vbb = __shfl(rb, tt, 64);
      }
      const int dim0 = (D == 64) ? 8 * (c16 & 7) : VDIM * c16;
      const half_t* vr = vb + (int64_t)va * p.v_sa + (int64_t)vbb * p.v_sb + dim0;
#pragma unroll
      for (int j = 0; j < VLD; ++j) vreg[i][j] = vv ? ld16(vr + 8 * j) : uint4_t{0, 0, 0, 0};
    }

    // ---- scores ----------------------------------------------------------
    float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) sacc = mfma16x16x32(as_half8(kreg[s]), qf[s], sacc);

    float t[4];
    if constexpr (MAGIC) {
      // |k|^2 of token c16 (K-lane layout), then fetch for tokens 4R + r.
      float ks = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) ks = dot2(kreg[s][j], kreg[s][j], ks);
      ks = rows_sum(ks);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tt = 4 * R + r;
        const float kn = sqrtf(__shfl(ks, tt, 64));
        const float dotp = sacc[r];
        float cosv = dotp / (q_norm * kn + 1e-8f);
        cosv = fminf(fmaxf(cosv, -1.0f + 1e-7f), 1.0f - 1e-7f);
        double pi = 1.0 - (1.0 / M_PI) * acos((double)cosv);
        pi = fmin(fmax(pi, 0.0), 1.0);
        const double xk = pow(pi, (double)lsh_k);
        double om = fmin(fmax(1.0 - xk, 0.0), 1.0);
        const double L = (double)lsh_l;
        double u = 1.0 - pow(om, L) - L * xk * pow(om, L - 1.0);
        u = fmax(u, 1e-10);
        const float sc = dotp * p.inv_sqrt_d - (float)log(u);
        t[r] = ((vmask >> tt) & 1) ? sc * kLog2e : AKT_NEG_INF;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        t[r] = ((vmask >> (4 * R + r)) & 1) ? sacc[r] * p.qk_scale : AKT_NEG_INF;
    }

    // ---- online softmax (head c16) -------------------------------------
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

    // ---- P.V -------------------------------------------------------------
    uint32_t vp[NPAIR][VDIM];
#pragma unroll
    for (int q2 = 0; q2 < NPAIR; ++q2)
#pragma unroll
      for (int j = 0; j < VLD; ++j)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t a = vreg[2 * q2][j][w], bq = vreg[2 * q2 + 1][j][w];
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
  }

  // ---- wave reduction --------------------------------------------------
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

  // ---- workgroup merge + output ----------------------------------------
  for (int idx = tid; idx < GT * D; idx += kThreads) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = AKT_NEG_INF;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.f, E = 0.f, O = 0.f;
    if (M != AKT_NEG_INF) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = fast_exp2(sm_m[w][h] - M);
        L += f * sm_l[w][h];
        E += f * sm_e[w][h];
        O += f * sm_o[w][h][d];
      }
    }
    if (h >= nh) continue;
    if (direct) {
      const int64_t row = (int64_t)b * p.Hq + hq0 + h;
      p.o[row * D + d] = (half_t)(L > 0.f ? O / L : 0.f);
      if (d == 0 && p.lse) p.lse[row] = E > 0.f ? (M + log2f(E)) * kLn2 : AKT_NEG_INF;
    } else {
      p.part_o[(pidx * GT + h) * D + d] = O;
      if (d == 0) {
        float* ml = p.part_ml + (pidx * GT + h) * 4;
        ml[0] = M;
        ml[1] = L;
        ml[2] = E;
        ml[3] = 0.f;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Log-sum-exp combine of split partials.
// ---------------------------------------------------------------------------
template <int D, int GT, int MODE>
__global__ __launch_bounds__(kThreads) void split_combine_kernel(SplitParams p) {
  constexpr bool SPARSE = (MODE == kModeSparseDense || MODE == kModeSparsePaged);
  int b, hq0, nh, nch;
  int64_t first, step;
  if constexpr (SPARSE) {
    const int u = blockIdx.x;
    b = u / p.Hq;
    hq0 = u - b * p.Hq;
    nh = 1;
    nch = p.n_split;
    if (nch == 1) return;
    first = (int64_t)u * p.n_split;
    step = 1;
  } else {
    b = blockIdx.x;
    const int y = blockIdx.y;
    const int kvh = y / p.n_hg;
    const int hg = y - kvh * p.n_hg;
    hq0 = kvh * p.G + hg * GT;
    nh = min(GT, p.G - hg * GT);
    int cs;
    if constexpr (MODE == kModeDense) {
      nch = (p.S + p.chunk - 1) / p.chunk;
      cs = b * nch;
    } else {
      chunk_span(p, b, cs, nch);
    }
    if (nch == 1) return;
    first = (int64_t)cs * gridDim.y + y;
    step = gridDim.y;
  }
  for (int idx = threadIdx.x; idx < nh * D; idx += kThreads) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = AKT_NEG_INF;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, p.part_ml[((first + c * step) * GT + h) * 4]);
    float L = 0.f, E = 0.f, O = 0.f;
    if (M != AKT_NEG_INF) {
      for (int c = 0; c < nch; ++c) {
        const int64_t pi = (first + c * step) * GT + h;
        const float f = fast_exp2(p.part_ml[pi * 4] - M);
        L += f * p.part_ml[pi * 4 + 1];
        E += f * p.part_ml[pi * 4 + 2];
        O += f * p.part_o[pi * D + d];
      }
    }
    const int64_t row = (int64_t)b * p.Hq + hq0 + h;
    p.o[row * D + d] = (half_t)(L > 0.f ? O / L : 0.f);
    if (d == 0 && p.lse) p.lse[row] = E > 0.f ? (M + log2f(E)) * kLn2 : AKT_NEG_INF;
  }
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

template <int D, int GT, int MODE, bool ALIGNED, bool MAGIC>
int launch_t(const SplitParams& p, dim3 grid, dim3 cgrid, hipStream_t st) {
  int rc = AKT_OK;
  if (grid.x > 0 && grid.y > 0) {
    KernelTimer timer(st);
    hipLaunchKernelGGL((split_kernel<D, GT, MODE, ALIGNED, MAGIC>), grid, dim3(kThreads), 0, st, p);
    timer.stop();
    rc = check_launch("split_kernel");
    if (rc) return rc;
  }
  if (cgrid.x > 0 && cgrid.y > 0) {
    hipLaunchKernelGGL((split_combine_kernel<D, GT, MODE>), cgrid, dim3(kThreads), 0, st, p);
    rc = check_launch("split_combine_kernel");
  }
  return rc;
}

template <int D, int MODE, bool ALIGNED, bool MAGIC>
int launch_gt(int gt, const SplitParams& p, dim3 grid, dim3 cgrid, hipStream_t st) {
  if constexpr (MODE == kModeSparseDense || MODE == kModeSparsePaged) {
    return launch_t<D, 1, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
  } else {
    switch (gt) {
      case 1: return launch_t<D, 1, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
      case 2: return launch_t<D, 2, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
      case 4: return launch_t<D, 4, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
      case 8: return launch_t<D, 8, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
      case 16:
        if constexpr (D != 256) return launch_t<D, 16, MODE, ALIGNED, MAGIC>(p, grid, cgrid, st);
        break;
    }
    return set_error(AKT_ERR_UNSUPPORTED, "no decode kernel for %d heads per unit", gt);
  }
}

template <int MODE, bool ALIGNED, bool MAGIC>
int launch_d(int D, int gt, const SplitParams& p, dim3 grid, dim3 cgrid, hipStream_t st) {
  switch (D) {
    case 64: return launch_gt<64, MODE, ALIGNED, MAGIC>(gt, p, grid, cgrid, st);
    case 128: return launch_gt<128, MODE, ALIGNED, MAGIC>(gt, p, grid, cgrid, st);
    case 256: return launch_gt<256, MODE, ALIGNED, MAGIC>(gt, p, grid, cgrid, st);
  }
  return set_error(AKT_ERR_UNSUPPORTED, "head_dim %d not supported (64, 128, 256)", D);
}

// Automatic chunk length for dense / paged caches: aim for ~4096 workgroups.
int64_t auto_chunk(int64_t total_tokens, int64_t units) {
  int64_t c = ceil_div(total_tokens * units, 4096);
  c = round_up(c < 64 ? 64 : c, 64);
  return c > 4096 ? 4096 : c;
}

int64_t auto_splits(int64_t rows, int64_t l_max) {
  int64_t s = ceil_div(1024, rows > 0 ? rows : 1);
  const int64_t cap = ceil_div(l_max > 0 ? l_max : 1, 64);
  if (s > cap) s = cap;
  return s < 1 ? 1 : s;
}

size_t split_ws_bytes(int64_t parts, int gt, int64_t D) {
  return (size_t)parts * gt * (D + 4) * sizeof(float);
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
  const int64_t n_hg = ceil_div(G, gt);
  const int64_t units = batch * num_kv_heads * n_hg;
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(seq_len * batch, num_kv_heads * n_hg);
  const int64_t nch = ceil_div(seq_len, chunk);
  return nch > 1 ? split_ws_bytes(units * nch, gt, head_dim) : 0;
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
  AKT_CHECK(chunk_tokens >= 0 && chunk_tokens % 64 == 0, "chunk_tokens must be a multiple of 64");
  if (batch == 0) return AKT_OK;
  const int D = (int)head_dim;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, D);
  const int n_hg = (int)ceil_div(G, gt);
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens
                                         : auto_chunk(seq_len * batch, num_kv_heads * n_hg);
  const int64_t nch = ceil_div(seq_len, chunk);
  const int64_t Y = num_kv_heads * n_hg;
  const size_t need = nch > 1 ? split_ws_bytes(batch * Y * nch, gt, D) : 0;
  if (need && (!workspace || workspace_bytes < need))
    return set_error(AKT_ERR_WORKSPACE, "workspace of %zu bytes required", need);

  SplitParams p = {};
  p.q = (const half_t*)q;
  p.kbase = (const half_t*)k;
  p.vbase = (const half_t*)v;
  p.o = (half_t*)o;
  p.lse = lse;
  p.part_o = (float*)workspace;
  p.part_ml = p.part_o + (need ? (size_t)batch * Y * nch * gt * D : 0);
  p.q_sb = q_stride[0];
  p.q_sh = q_stride[1];
  p.k_sa = k_stride[2]; p.k_sb = 0; p.k_batch = k_stride[0]; p.k_head = k_stride[1];
  p.v_sa = v_stride[2]; p.v_sb = 0; p.v_batch = v_stride[0]; p.v_head = v_stride[1];
  p.B = (int)batch; p.Hq = (int)num_q_heads; p.Hkv = (int)num_kv_heads; p.G = G;
  p.S = (int)seq_len;
  p.n_hg = n_hg;
  p.chunk = (int)chunk;
  p.qk_scale = softmax_scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;
  // nch == 0 (empty cache): only the combine pass runs and writes 0 / -inf.
  dim3 grid((unsigned)(batch * nch), (unsigned)Y);
  dim3 cgrid(nch == 1 ? 0u : (unsigned)batch, (unsigned)Y);
  return launch_d<kModeDense, false, false>(D, gt, p, grid, cgrid, st);
}

// ----------------------------- paged decode --------------------------------
static int64_t paged_grid_x(int64_t total_pages, int64_t page_size, int64_t chunk, int64_t batch) {
  return ceil_div(total_pages * page_size, chunk) + batch;
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
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(total_pages * page_size, Y);
  return split_ws_bytes(paged_grid_x(total_pages, page_size, chunk, batch) * Y, gt, head_dim);
}

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
  int rc = check_common(batch, num_q_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  AKT_CHECK(page_size > 0 && page_size < (1 << 20), "page_size out of range");
  AKT_CHECK(total_pages >= 0 && num_pool_pages >= 0 && total_pages * page_size < (1ll << 31),
            "page counts out of range");
  AKT_CHECK(q_stride[3] == 1 && kv_stride[4] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 3) && rows_aligned16(kv_cache, kv_stride, 4) && aligned16(o),
            "tensors must have 16-byte aligned rows");
  AKT_CHECK(chunk_tokens >= 0 && chunk_tokens % 64 == 0, "chunk_tokens must be a multiple of 64");
  if (batch == 0) return AKT_OK;
  const int D = (int)head_dim;
  const int G = (int)(num_q_heads / num_kv_heads);
  const int gt = pick_gt(G, D);
  const int n_hg = (int)ceil_div(G, gt);
  const int64_t Y = num_kv_heads * n_hg;
  const int64_t chunk = chunk_tokens > 0 ? chunk_tokens : auto_chunk(total_pages * page_size, Y);
  const int64_t gx = paged_grid_x(total_pages, page_size, chunk, batch);
  const size_t need = split_ws_bytes(gx * Y, gt, D);
  if (!workspace || workspace_bytes < need)
    return set_error(AKT_ERR_WORKSPACE, "workspace of %zu bytes required", need);

  SplitParams p = {};
  p.q = (const half_t*)q;
  p.kbase = (const half_t*)kv_cache;
  p.vbase = (const half_t*)kv_cache + kv_stride[1];
  p.indptr = kv_page_indptr;
  p.indices = kv_page_indices;
  p.last_len = kv_last_page_len;
  p.o = (half_t*)o;
  p.lse = lse;
  p.part_o = (float*)workspace;
  p.part_ml = p.part_o + (size_t)gx * Y * gt * D;
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
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)gx, (unsigned)Y);
  dim3 cgrid((unsigned)batch, (unsigned)Y);
  if (page_size % 16 == 0) return launch_d<kModePaged, true, false>(D, gt, p, grid, cgrid, st);
  return launch_d<kModePaged, false, false>(D, gt, p, grid, cgrid, st);
}

// ----------------------------- sparse decode -------------------------------
extern "C" size_t akt_sparse_decode_workspace_size(int64_t batch, int64_t num_q_heads,
                                                   int64_t head_dim, int64_t l_max,
                                                   int64_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || !head_dim_ok(head_dim)) return 0;
  const int64_t rows = batch * num_q_heads;
  const int64_t ns = num_splits > 0 ? num_splits : auto_splits(rows, l_max);
  return ns > 1 ? split_ws_bytes(rows * ns, 1, head_dim) : 0;
}

namespace {

int sparse_common(SplitParams& p, const void* q, const int32_t* sparse_ind,
                  const int32_t* sparse_nnz, void* o, float* lse, int64_t batch,
                  int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t l_max,
                  const int64_t q_stride[4], const int64_t ind_stride[2],
                  const int64_t nnz_stride[2], int64_t num_splits, void* workspace,
                  size_t workspace_bytes, int64_t& ns_out) {
  int rc = check_common(batch, num_q_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  AKT_CHECK(l_max >= 0 && l_max < (1ll << 31), "l_max out of range");
  AKT_CHECK(q_stride[3] == 1, "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 2) && aligned16(o), "tensors must have 16-byte aligned rows");
  AKT_CHECK(num_splits >= 0, "num_splits must be >= 0");
  const int64_t rows = batch * num_q_heads;
  const int64_t ns = num_splits > 0 ? num_splits : auto_splits(rows, l_max);
  const size_t need = ns > 1 ? split_ws_bytes(rows * ns, 1, head_dim) : 0;
  if (need && (!workspace || workspace_bytes < need))
    return set_error(AKT_ERR_WORKSPACE, "workspace of %zu bytes required", need);
  p.q = (const half_t*)q;
  p.sparse_ind = sparse_ind;
  p.sparse_nnz = sparse_nnz;
  p.o = (half_t*)o;
  p.lse = lse;
  p.part_o = (float*)workspace;
  p.part_ml = p.part_o + (need ? (size_t)rows * ns * head_dim : 0);
  p.q_sb = q_stride[0];
  p.q_sh = q_stride[1];
  p.ind_sb = ind_stride[0];
  p.ind_sh = ind_stride[1];
  p.nnz_sb = nnz_stride[0];
  p.nnz_sh = nnz_stride[1];
  p.B = (int)batch; p.Hq = (int)num_q_heads; p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.l_max = (int)l_max;
  p.n_split = (int)ns;
  ns_out = ns;
  return AKT_OK;
}

}  // namespace

extern "C" int akt_sparse_decode_fwd(const void* q, const void* k, const void* v,
                                     const int32_t* sparse_ind, const int32_t* sparse_nnz,
                                     void* o, float* lse, int64_t batch, int64_t num_q_heads,
                                     int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                     int64_t l_max, const int64_t q_stride[4],
                                     const int64_t k_stride[4], const int64_t v_stride[4],
                                     const int64_t ind_stride[2], const int64_t nnz_stride[2],
                                     float softmax_scale, int64_t num_splits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  clear_error();
  SplitParams p = {};
  int64_t ns = 0;
  int rc = sparse_common(p, q, sparse_ind, sparse_nnz, o, lse, batch, num_q_heads, num_kv_heads,
                         head_dim, l_max, q_stride, ind_stride, nnz_stride, num_splits,
                         workspace, workspace_bytes, ns);
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
  dim3 grid((unsigned)(rows * ns), 1);
  dim3 cgrid(ns > 1 ? (unsigned)rows : 0u, 1);
  return launch_d<kModeSparseDense, false, false>((int)head_dim, 1, p, grid, cgrid,
                                                  (hipStream_t)stream);
}

static int sparse_paged_impl(bool magic, const void* q, const void* kv_cache,
                             const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                             const int32_t* sparse_ind, const int32_t* sparse_nnz,
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
  int rc = sparse_common(p, q, sparse_ind, sparse_nnz, o, lse, batch, num_q_heads, num_kv_heads,
                         head_dim, l_max, q_stride, ind_stride, nnz_stride, num_splits,
                         workspace, workspace_bytes, ns);
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
  dim3 grid((unsigned)(rows * ns), 1);
  dim3 cgrid(ns > 1 ? (unsigned)rows : 0u, 1);
  hipStream_t st = (hipStream_t)stream;
  if (magic) return launch_d<kModeSparsePaged, false, true>((int)head_dim, 1, p, grid, cgrid, st);
  return launch_d<kModeSparsePaged, false, false>((int)head_dim, 1, p, grid, cgrid, st);
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
                           sparse_nnz, nullptr, nullptr, o, lse, batch, num_q_heads, num_kv_heads,
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
                           sparse_nnz, lsh_k, lsh_l, o, lse, batch, num_q_heads, num_kv_heads,
                           head_dim, page_size, num_pool_pages, l_max, q_stride, kv_stride,
                           ind_stride, nnz_stride, 1.0f / sqrtf((float)head_dim), num_splits,
                           workspace, workspace_bytes, stream);
}
