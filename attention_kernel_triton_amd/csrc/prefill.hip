// Causal / non-causal GQA flash-attention prefill for gfx950.
//
// Replaces the reference's Triton prefill kernels
//   prefill_flash_attention.py:18-335           (dense)
//   prefill_flash_attention_var_len_padding.py:109-341  (right-padded var-len)
// with an MFMA kernel designed around CDNA4's v_mfma_f32_32x32x16_f16.
//
// Tiling.  A 256-thread workgroup owns 128 query rows of one (batch, q head);
// wave w owns rows 32w..32w+31.  Keys stream through LDS in 64-key tiles:
//   sK  : K tile, row-major [key][dim] (row padded by 16 bytes)
//   sVt : V tile transposed [dim][key] (row padded by 16 bytes) with the key
//         order permuted so that each MFMA operand read is one 16-byte access.
// Both products are computed transposed so that each lane owns one query row:
//   S^T = K . Q^T    (A = K from LDS, B = Q^T held in registers)
//   O^T = V^T . P^T  (A = V^T from LDS, B = P^T straight from the S^T registers)
// With the 32x32 result layout, lane l holds query row l & 31 and 16 key (or
// dim) slots; the two 32-lane halves hold complementary slots, so the row max
// and row sum need one exchange between lane l and l ^ 32.
//
// Softmax.  Scores are scaled by softmax_scale * log2(e) and exponentiated
// with v_exp_f32.  The running max is only raised when a tile's max exceeds it
// by more than kRescaleSlack (in log2 units); otherwise the stale max is kept,
// which bounds P by 2^kRescaleSlack and skips the O rescale.  P is rounded to
// fp16 for the P.V product (as the reference does at prefill_flash_attention.py:94)
// and the normaliser sums the same rounded values.
//
// Masking uses a select (score = -inf), not an additive -1e6 as in the
// reference (prefill_flash_attention.py:76), so non-finite padding never leaks.
// In var-len causal mode the K/V rows at or beyond a sequence's length are
// staged as zeros, so padding cannot reach valid rows through P.V either.
#include <math.h>

#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {

namespace {

constexpr int kPThreads = 256;
constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr float kRescaleSlack = 8.0f;
#define AKT_P_NEG_INF (-__builtin_inff())

struct PrefillParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  const void* varlen;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, G, S;
  int varlen_bits;
  int n_qblk;    // query blocks per head
  int xcd_map;   // 1: group kv heads per XCD (requires (B*Hkv) % 8 == 0)
  float qk_scale;  // softmax_scale * log2(e)
};

// Key position inside a 64-key sVt row: swaps bits 2 and 3 of the key index so
// that the 8 keys one lane feeds to a 32x32x16 MFMA are contiguous.
__device__ __forceinline__ int vt_pos(int key) {
  return (key & ~15) | ((key & 4) << 1) | ((key & 8) >> 1) | (key & 3);
}

// Workgroup -> (batch, q head, query block).  Causal work is issued heaviest
// block first; with xcd_map the workgroups of one kv head land on one XCD
// (workgroup i is dispatched to XCD i % 8) so its L2 serves the G query heads.
__device__ __forceinline__ void map_block(const PrefillParams& p, bool causal, int& b, int& h,
                                          int& qb) {
  const int pid = blockIdx.x;
  const int nheads = p.B * p.Hq;
  int rank, head;
  if (p.xcd_map) {
    const int xcd = pid & 7;
    const int j = pid >> 3;
    const int nk = (p.B * p.Hkv) >> 3;  // kv groups per XCD
    const int per_rank = nk * p.G;
    rank = j / per_rank;
    const int rem = j - rank * per_rank;
    const int kl = rem / p.G;
    const int g = rem - kl * p.G;
    const int kg = kl * 8 + xcd;  // global kv group = b * Hkv + kvh
    head = kg * p.G + g;          // = b * Hq + kvh * G + g
  } else {
    rank = pid / nheads;
    head = pid - rank * nheads;
  }
  b = head / p.Hq;
  h = head - b * p.Hq;
  qb = causal ? (p.n_qblk - 1 - rank) : rank;
}

template <int D, bool CAUSAL, bool VARLEN>
__global__ __launch_bounds__(kPThreads) void prefill_kernel(PrefillParams p) {
  constexpr int KS = D / 16;       // MFMA k-steps over the head dim
  constexpr int HALF = D / 2;      // head dims per lane half in S^T operands
  constexpr int KROW = D + 8;      // sK row pitch (halfs)
  constexpr int VROW = kBN + 8;    // sVt row pitch (halfs)
  constexpr int NT = D / 32;       // 32-dim output tiles
  constexpr int K_CHUNKS = kBN * D / 8;         // 16-byte chunks per K tile
  constexpr int V_PAIRS = (kBN / 2) * (D / 8);  // (key pair, 8 dims) chunks per V tile
  constexpr int K_PER_T = K_CHUNKS / kPThreads;
  constexpr int V_PER_T = V_PAIRS / kPThreads;
  static_assert(K_CHUNKS % kPThreads == 0 && V_PAIRS % kPThreads == 0, "tile split");

  __shared__ __attribute__((aligned(16))) half_t sK[kBN * KROW];
  __shared__ __attribute__((aligned(16))) half_t sVt[D * VROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int b, h, qb;
  map_block(p, CAUSAL, b, h, qb);
  const int S = p.S;
  int len = S;
  if constexpr (VARLEN) {
    long long lv = (p.varlen_bits == 64) ? ((const long long*)p.varlen)[b]
                                         : (long long)((const int*)p.varlen)[b];
    len = (int)(lv < 0 ? 0 : (lv > S ? S : lv));
  }
  // Rows are computed in 64-row blocks up to ceil(len / 64) * 64, as the
  // reference does (prefill_flash_attention_var_len_padding.py:185-187).
  const int row_lim = VARLEN ? min(S, ((len + 63) / 64) * 64) : S;
  const int q0 = qb * kBM;
  if (q0 >= row_lim) return;
  const int kvh = h / p.G;

  const half_t* __restrict__ Qh = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const half_t* __restrict__ Kh = p.k + (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh;
  const half_t* __restrict__ Vh = p.v + (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh;
  half_t* __restrict__ Oh = p.o + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;

  const int qw0 = q0 + 32 * wave;
  const int row = qw0 + l32;
  const bool wave_rows = qw0 < row_lim;

  // Q^T fragment: lane -> row, dims g*HALF + 8s + e.
  half8_t qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    uint4_t v = {0, 0, 0, 0};
    if (row < S) v = ld16(Qh + (int64_t)row * p.q_ss + g * HALF + 8 * s);
    qf[s] = as_half8(v);
  }

  // Keys this workgroup needs, and keys that must be staged as zeros.
  int kv_end = S;
  if constexpr (CAUSAL) kv_end = min(row_lim, q0 + kBM);
  const int key_lim = (VARLEN && CAUSAL) ? len : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  const int wave_kv_end = CAUSAL ? min(kv_end, qw0 + 32) : kv_end;

  float16_t oacc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[n][r] = 0.f;
  float m_run = AKT_P_NEG_INF;
  float l_part = 0.f;
  const float c = p.qk_scale;
  const uint32_t kOnes = 0x3c003c00u;

  // Staging registers for the next tile.
  uint4_t kst[K_PER_T];
  uint4_t vst[V_PER_T][2];
  auto load_tile = [&](int j) {
    const int kbase = j * kBN;
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int cidx = tid + i * kPThreads;
      const int key = cidx / (D / 8);
      const int dc = cidx - key * (D / 8);
      const int kg = kbase + key;
      kst[i] = (kg < key_lim) ? ld16(Kh + (int64_t)kg * p.k_ss + 8 * dc) : uint4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int cidx = tid + i * kPThreads;
      const int kp = cidx / (D / 8);
      const int dc = cidx - kp * (D / 8);
      const int kg = kbase + 2 * kp;
      vst[i][0] = (kg < key_lim) ? ld16(Vh + (int64_t)kg * p.v_ss + 8 * dc) : uint4_t{0, 0, 0, 0};
      vst[i][1] =
          (kg + 1 < key_lim) ? ld16(Vh + (int64_t)(kg + 1) * p.v_ss + 8 * dc) : uint4_t{0, 0, 0, 0};
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int cidx = tid + i * kPThreads;
      const int key = cidx / (D / 8);
      const int dc = cidx - key * (D / 8);
      *reinterpret_cast<uint4_t*>(&sK[key * KROW + 8 * dc]) = kst[i];
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int cidx = tid + i * kPThreads;
      const int kp = cidx / (D / 8);
      const int dc = cidx - kp * (D / 8);
      const int pos = vt_pos(2 * kp);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t a = vst[i][0][w], bb = vst[i][1][w];
        *reinterpret_cast<uint32_t*>(&sVt[(8 * dc + 2 * w) * VROW + pos]) = pair_lo(a, bb);
        *reinterpret_cast<uint32_t*>(&sVt[(8 * dc + 2 * w + 1) * VROW + pos]) = pair_hi(a, bb);
      }
    }
  };

  if (n_tiles > 0) load_tile(0);
  for (int j = 0; j < n_tiles; ++j) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (j + 1 < n_tiles) load_tile(j + 1);

    const int kt0 = j * kBN;
    if (!wave_rows || kt0 >= wave_kv_end) continue;  // wave-uniform

    // ---- S^T = K . Q^T for the two 32-key halves of the tile ------------
    float16_t sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[t][r] = 0.f;
      const half_t* kr = &sK[(32 * t + l32) * KROW + g * HALF];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const half8_t a = as_half8(*reinterpret_cast<const uint4_t*>(kr + 8 * s));
        sacc[t] = mfma32x32x16(a, qf[s], sacc[t]);
      }
    }

    // ---- mask -----------------------------------------------------------
    const bool need_mask = (CAUSAL && kt0 + kBN - 1 > qw0) || (kt0 + kBN > S);
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt0 + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = (key < S) && (!CAUSAL || key <= row);
          if (!ok) sacc[t][r] = AKT_P_NEG_INF;
        }
    }

    // ---- online softmax (row = l32) -------------------------------------
    float mx = sacc[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
    mx = fmaxf(mx, shfl_xor_f(mx, 32)) * c;
    if (__any(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_new > m_run) ? fast_exp2(m_run - m_new) : 1.0f;
      l_part *= alpha;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[n][r] *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == AKT_P_NEG_INF) ? 0.f : m_run;
    uint32_t pk[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(__builtin_fmaf(sacc[t][r], c, -m_use));
        const float p1 = fast_exp2(__builtin_fmaf(sacc[t][r + 1], c, -m_use));
        pk[t][r >> 1] = pack_half2(p0, p1);
        l_part = dot2(pk[t][r >> 1], kOnes, l_part);
      }

    // ---- O^T += V^T . P^T -------------------------------------------------
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const half8_t bop =
            as_half8(uint4_t{pk[t][4 * u], pk[t][4 * u + 1], pk[t][4 * u + 2], pk[t][4 * u + 3]});
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const half8_t a = as_half8(*reinterpret_cast<const uint4_t*>(
              &sVt[(32 * n + l32) * VROW + 32 * t + 16 * u + 8 * g]));
          oacc[n] = mfma32x32x16(a, bop, oacc[n]);
        }
      }
  }

  if (!wave_rows || row >= row_lim) return;
  const float l_row = l_part + shfl_xor_f(l_part, 32);
  const float inv = l_row > 0.f ? 1.0f / l_row : 0.f;
  half_t* orow = Oh + (int64_t)row * p.o_ss;
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      half4_t hv;
#pragma unroll
      for (int r = 0; r < 4; ++r) hv[r] = (half_t)(oacc[n][4 * q4 + r] * inv);
      *reinterpret_cast<half4_t*>(orow + 32 * n + 8 * q4 + 4 * g) = hv;
    }
}

template <int D, bool CAUSAL, bool VARLEN>
int launch(const PrefillParams& p, unsigned grid, hipStream_t st) {
  KernelTimer timer(st);
  hipLaunchKernelGGL((prefill_kernel<D, CAUSAL, VARLEN>), dim3(grid), dim3(kPThreads), 0, st, p);
  timer.stop();
  return check_launch("prefill_kernel");
}

template <int D>
int launch_d(bool causal, bool varlen, const PrefillParams& p, unsigned grid, hipStream_t st) {
  if (causal) return varlen ? launch<D, true, true>(p, grid, st) : launch<D, true, false>(p, grid, st);
  return varlen ? launch<D, false, true>(p, grid, st) : launch<D, false, false>(p, grid, st);
}

}  // namespace
}  // namespace akt

using namespace akt;

extern "C" int akt_prefill_fwd(const void* q, const void* k, const void* v, void* o, int64_t batch,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                               int64_t head_dim, const int64_t q_stride[4],
                               const int64_t k_stride[4], const int64_t v_stride[4],
                               const int64_t o_stride[4], float softmax_scale, int causal,
                               const void* varlen, int varlen_bits, void* stream) {
  clear_error();
  AKT_CHECK(batch >= 0 && num_q_heads > 0 && num_kv_heads > 0, "batch/head counts must be positive");
  AKT_CHECK(num_q_heads % num_kv_heads == 0,
            "num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)", (long long)num_q_heads,
            (long long)num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return set_error(AKT_ERR_UNSUPPORTED, "prefill head_dim %lld not supported (64, 128)",
                     (long long)head_dim);
  AKT_CHECK(seq_len >= 0 && seq_len < (1ll << 30), "seq_len out of range");
  AKT_CHECK(q_stride[3] == 1 && k_stride[3] == 1 && v_stride[3] == 1 && o_stride[3] == 1,
            "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 3) && rows_aligned16(k, k_stride, 3) &&
                rows_aligned16(v, v_stride, 3) && rows_aligned16(o, o_stride, 3),
            "tensors must have 16-byte aligned rows");
  AKT_CHECK(!varlen || varlen_bits == 32 || varlen_bits == 64, "varlen_bits must be 32 or 64");
  AKT_CHECK(softmax_scale > 0.f, "softmax_scale must be positive");
  if (batch == 0 || seq_len == 0) return AKT_OK;

  PrefillParams p = {};
  p.q = (const half_t*)q;
  p.k = (const half_t*)k;
  p.v = (const half_t*)v;
  p.o = (half_t*)o;
  p.varlen = varlen;
  p.varlen_bits = varlen_bits;
  p.q_sb = q_stride[0]; p.q_sh = q_stride[1]; p.q_ss = q_stride[2];
  p.k_sb = k_stride[0]; p.k_sh = k_stride[1]; p.k_ss = k_stride[2];
  p.v_sb = v_stride[0]; p.v_sh = v_stride[1]; p.v_ss = v_stride[2];
  p.o_sb = o_stride[0]; p.o_sh = o_stride[1]; p.o_ss = o_stride[2];
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.S = (int)seq_len;
  p.n_qblk = (int)ceil_div(seq_len, kBM);
  p.xcd_map = ((batch * num_kv_heads) % 8 == 0) ? 1 : 0;
  p.qk_scale = softmax_scale * kLog2e;
  const int64_t grid = batch * num_q_heads * p.n_qblk;
  AKT_CHECK(grid < (1ll << 31), "problem too large");
  const bool is_causal = causal != 0;
  const bool is_var = varlen != nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (head_dim == 64) return launch_d<64>(is_causal, is_var, p, (unsigned)grid, st);
  return launch_d<128>(is_causal, is_var, p, (unsigned)grid, st);
}
