// Causal / non-causal GQA flash-attention prefill for gfx950.
//
// Replaces the reference's Triton prefill kernels
//   prefill_flash_attention.py:18-335                   (dense)
//   prefill_flash_attention_var_len_padding.py:109-341  (right-padded var-len)
// with an MFMA kernel designed around CDNA4's v_mfma_f32_32x32x16_f16 (or its
// bf16 form for bf16 tensors) and the transposing LDS read (ds_read_b64_tr_b16).
//
// Work decomposition.  A 256-thread workgroup serves one (batch, kv head) and
// four "slots"; slot f = (query head f % G, row block f / G) of that kv head's
// G query heads (64-row blocks at D = 64 and in the long-sequence D = 128
// instance, 32-row blocks otherwise).  With G a multiple of 4 the four waves
// are four query heads at the same rows: they share every staged K/V tile and
// have identical causal extents.  With 64-row blocks each wave owns its rows
// as two 32-row MFMA blocks that share every K and V fragment read from LDS
// (see rblocks_for).
//
// K/V staging.  Each tile of K and V (64 keys with two row blocks, else 32) goes
// global -> registers -> one of four LDS tile buffers: while tile j is
// computed, tile j + 1 is already
// published, tile j + 2 is being written and tile j + 3 is in flight from
// HBM, and one barrier per tile both publishes a tile and retires tile j - 2's
// buffer.  (Direct global -> LDS copies would be waited for before every
// transposing LDS read, which defeats the prefetch.)  Rows are stored without
// padding; 16-byte chunk c of row r sits at chunk position c ^ tswz<D>(r).
// gfx950's LDS has 64 four-byte banks; a 16-byte access serves 16 lanes per
// cycle and an 8-byte one 32 (measured with SQ_LDS_BANK_CONFLICT on single
// access patterns).  The swizzle keeps the 16-byte K reads (16 consecutive
// rows, one chunk each), the transposing V reads (4 rows x 4 chunks x 2 halves
// per 32 lanes) and the tile stores free of bank conflicts at every head dim.
// Rows past the keys a tile may use fall outside the tile's
// buffer-resource range and read as zeros, so every staged value is finite
// and no read leaves the tensor.
//
// Per 32-key step t a wave runs, with no dependence between the three parts:
//   O^T += V^T . P(t-1)^T   A = V^T via ds_read_b64_tr_b16, B = the previous
//                           step's probabilities straight from registers
//   S(t+1)^T = K . Q^T      A = K rows (16-byte LDS reads), B = Q^T in registers
//   softmax of S(t)^T       VALU / transcendental work
// so the MFMA pipe and the VALU work of one wave overlap.  Computing both
// products transposed makes each lane own one query row (lane & 31) of each
// 32-row block; the two 32-lane halves hold complementary key (or dim) slots,
// so row max / sum need one v_permlane32_swap.
//
// Softmax.  Scores are scaled by softmax_scale * log2(e) and exponentiated with
// v_exp_f32 against the running max as it stands; no per-step row max is
// taken.  The running max starts at the row max of step 0.  Only when a row's
// sum over a step shows a probability above 2^kRescaleSlack (or a NaN) does
// the wave take a rare branch that computes the row max, raises the running
// max of the rows that exceed it by more than kRescaleSlack (log2 units),
// rescales their normaliser and O (after the step's P.V(t-1) has been
// accumulated) and recomputes P.  So P
// stays below 32 * 2^kRescaleSlack and the O rescale is almost never run.  P
// is rounded to fp16 for P.V (as the reference does at
// prefill_flash_attention.py:94) and the normaliser sums the same rounded
// values, each row on its own (a NaN query row leaves every other row
// exact, as in the reference).
//
// Masking uses a select (score = -inf), not the reference's additive -1e6
// (prefill_flash_attention.py:76), so non-finite padding never leaks.  In
// var-len causal mode the K/V rows at or beyond a sequence's length are never
// staged (zeros are read in their place), so padding cannot reach valid rows
// through P.V either.
#include <float.h>
#include <math.h>

#include <cmath>

#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {

// Kernel arguments (shared by both translation units of this file).
struct PrefillParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  const void* varlen;
  float* lse;  // optional [B, Hq, S] natural-log normaliser
  int64_t lse_sb, lse_sh, lse_ss;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, G, S;
  int varlen_bits;
  int n_rb;      // query row blocks (slots of one head) per sequence
  int n_sg;      // slot groups (workgroups) per (batch, kv head)
  int grid1d;    // 1: linear grid (a dimension past 65535); 0: grid (Hkv, B, n_sg)
  int fast_div;  // 1: G * n_rb + kSlots < 2^22, slot / G through g_inv
  float g_inv;   // 1 / G
  float qk_scale;  // |softmax_scale| * log2(e), at least FLT_MIN
  int neg_q;       // 1: softmax_scale < 0, computed as (-Q) K^T at |softmax_scale|
};

namespace {

constexpr int kPThreads = 256;
constexpr int kSlots = 4;   // waves per workgroup
constexpr int kNBuf = 4;    // LDS tile buffers
// 32-row MFMA blocks per wave, query rows per slot, keys per staged tile and
// waves per SIMD of an instance: two blocks and 64-key tiles at D = 64 (two
// waves per SIMD in 237 VGPRs); from D = 128 one block and 32-key tiles.  At
// D = 128 that holds a wave in 210 VGPRs and a workgroup's four K + V buffers
// in 64 KB, so two waves share each SIMD.  The LONG instance of D = 128 (for
// sequences of kLongRowsD128 rows or more) takes two blocks and 64-key tiles
// at one wave per SIMD (registers and AGPRs past 256, 128 KB of LDS): it is
// 4-6% slower at 1024 rows and 3.5-5% faster from 4096, where each
// workgroup's longer walk amortises its start.  At D = 192 and 256 the
// register budget allows one wave per SIMD either way.
__host__ __device__ constexpr bool two_blocks(int D, bool LONG) {
  return D == 64 || (D == 128 && LONG);
}
__host__ __device__ constexpr int rblocks_for(int D, bool LONG) { return two_blocks(D, LONG) ? 2 : 1; }
__host__ __device__ constexpr int rows_for(int D, bool LONG) { return 32 * rblocks_for(D, LONG); }
__host__ __device__ constexpr int tile_keys_for(int D, bool LONG) {
  return two_blocks(D, LONG) ? 64 : 32;
}
__host__ __device__ constexpr int waves_per_simd(int D, bool LONG) {
  return (D == 64 || (D == 128 && !LONG)) ? 2 : 1;
}
constexpr int kLongRowsD128 = 4096;
constexpr float kRescaleSlack = 8.0f;
// Largest row sum of one 32-key step that lets P stay unchecked: below it
// every probability is under 32 * 2^kRescaleSlack, far inside fp16's range;
// above it some probability exceeds 2^kRescaleSlack.
constexpr float kStepSumLimit = 32.0f * 256.0f;
static_assert(kRescaleSlack == 8.0f, "kStepSumLimit assumes a slack of 8");
#define AKT_P_NEG_INF (-__builtin_inff())



// Operand element type of a kernel instance: fp16 (v_mfma_f32_32x32x16_f16,
// P rounded to fp16 as the reference does) or bf16 (the bf16 MFMA, P rounded
// to bf16, since both MFMA operands share one type).  Global loads and the
// LDS staging move raw 16-byte chunks and do not depend on it.
template <bool BF16>
struct Elt {
  typedef half8_t v8;
  static constexpr uint32_t kOnes = 0x3c003c00u;  // (1, 1)
  static __device__ __forceinline__ v8 as8(uint4_t u) { return __builtin_bit_cast(v8, u); }
  static __device__ __forceinline__ float16_t mfma(v8 a, v8 b, float16_t c) {
    return mfma32x32x16(a, b, c);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_half2(lo, hi); }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return ::akt::dot2(a, b, c);
  }
};
template <>
struct Elt<true> {
  typedef bf16x8_t v8;
  static constexpr uint32_t kOnes = 0x3f803f80u;  // (1, 1)
  static __device__ __forceinline__ v8 as8(uint4_t u) { return __builtin_bit_cast(v8, u); }
  static __device__ __forceinline__ float16_t mfma(v8 a, v8 b, float16_t c) {
    return mfma32x32x16_bf16(a, b, c);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return dot2_bf16(a, b, c);
  }
};

// Chunk-position swizzle of a K / V tile row (see the header comment); a
// function of r mod 16, with tswz(r + 8) = tswz(r) ^ 2.
// - 64- and 192-dim rows (128 / 384 bytes) start on bank 0 or 32 by row
//   parity: over 16 consecutive rows the even rows' values are a permutation
//   of 0..7, and so are the odd rows' (K reads), and rows 4i + j and 4i + j + 2
//   differ in bit 2 (V reads: their 4-chunk blocks land in different halves).
// - 128- and 256-dim rows (256 / 512 bytes) all start on bank 0: 16
//   consecutive rows get a permutation of 0..15, and rows 4i..4i+3 differ in
//   bits 2..3.
template <int D>
__device__ __forceinline__ int tswz(int r) {
  if constexpr (D == 64 || D == 192) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return ((r & 3) << 2) | ((r >> 2) & 3);
}
// Chunk-position swizzle of the epilogue's O staging rows.
__device__ __forceinline__ int eswz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// Workgroup -> (batch, kv head, slot group).  The linear workgroup id is
// kvh + Hkv (b + B rank): causal work is issued heaviest slot group (lowest
// rank) first, and with B * Hkv a multiple of 8 every workgroup of a kv head
// lands on XCD (b Hkv + kvh) % 8 (workgroup i is dispatched to XCD i % 8), so
// one L2 serves all of them.  The grid (Hkv, B, n_sg) hands out the three
// indices without divisions; a linear grid (when a dimension exceeds 65535)
// derives them.
__device__ __forceinline__ void map_block(const PrefillParams& p, bool causal, int& b, int& kvh,
                                          int& sg) {
  int rank;
  if (p.grid1d) {
    const int pid = blockIdx.x;
    const int ngroups = p.B * p.Hkv;
    rank = pid / ngroups;
    const int kg = pid - rank * ngroups;
    b = kg / p.Hkv;
    kvh = kg - b * p.Hkv;
  } else {
    kvh = blockIdx.x;
    b = blockIdx.y;
    rank = blockIdx.z;
  }
  sg = causal ? (p.n_sg - 1 - rank) : rank;
}

// n / d for 0 <= n < 2^22 and d >= 1, given inv = 1 / d rounded to float:
// the float estimate is within one of the quotient, and one correction step
// makes it exact.  (n / d through the integer divide sequence costs several
// dependent VALU-to-SALU round trips at the start of every workgroup.)
__device__ __forceinline__ int div_small(int n, int d, float inv) {
  int q = (int)((float)n * inv);
  const int r = n - q * d;
  q += (r >= d ? 1 : 0) - (r < 0 ? 1 : 0);
  return q;
}

template <int D, bool CAUSAL, bool VARLEN, bool BF16, bool LONG>
__global__ __launch_bounds__(kPThreads)
__attribute__((amdgpu_waves_per_eu(waves_per_simd(D, LONG), 2)))
void prefill_kernel(PrefillParams p) {
  typedef Elt<BF16> E;
  typedef typename E::v8 v8;
  static_assert(!LONG || D == 128, "only D = 128 has a long-sequence instance");
  constexpr int NRB = rblocks_for(D, LONG);    // 32-row MFMA blocks per wave
  constexpr int kRows = rows_for(D, LONG);     // query rows per slot
  constexpr int kBN = tile_keys_for(D, LONG);  // keys per staged tile
  constexpr int SPT = kBN / 32;           // 32-key steps per tile
  constexpr int KS = D / 16;              // MFMA k-steps over the head dim
  constexpr int HALF = D / 2;             // head dims per lane half in S^T operands
  constexpr int NT = D / 32;              // 32-dim output tiles
  constexpr int CPR = D / 8;              // 16-byte chunks per K/V row
  constexpr int ROWB = D * 2;             // bytes per K/V row
  constexpr int TILEB = kBN * ROWB;       // bytes per K (or V) tile
  constexpr int BUFB = 2 * TILEB;         // bytes per tile buffer (K then V)
  static_assert((kBN * CPR) % kPThreads == 0, "tile split");
  // D = 64 reads the V fragments of step t + 1 at the end of step t, so P.V
  // starts without waiting for LDS; at D = 128 they would not fit in the
  // register budget and are read at the top of their step.
  constexpr bool kPrefetchV = (D == 64);

  __shared__ __attribute__((aligned(16))) char lds[kNBuf * BUFB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int b, kvh, sg;
  map_block(p, CAUSAL, b, kvh, sg);
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

  // This wave's slot and the workgroup's key range.
  auto div_g = [&](int n) { return uniform(p.fast_div ? div_small(n, p.G, p.g_inv) : n / p.G); };
  const int slot = sg * kSlots + wave;
  const int slot_q = div_g(slot);
  const int hl = slot - slot_q * p.G;
  const int r0 = slot_q * kRows;
  const bool active = slot < p.G * p.n_rb && r0 < row_lim;
  // Var-len: slots, and with them their row blocks, grow with the wave index,
  // so when the first slot's rows start past ceil(len / 64) * 64 no wave of
  // the workgroup has a row to compute, and it leaves before staging any tile
  // (workgroup-uniform).
  if constexpr (VARLEN) {
    if (div_g(sg * kSlots) * kRows >= row_lim) return;
  }
  int kv_end = S;
  if constexpr (CAUSAL) {
    // The workgroup's last valid slot has its largest row block.
    const int f_last = min(sg * kSlots + kSlots - 1, p.G * p.n_rb - 1);
    kv_end = min(row_lim, div_g(f_last) * kRows + kRows);
  }
  const int key_lim = (VARLEN && CAUSAL) ? len : S;  // rows at or past this are never staged
  // Tiles staged by the workgroup; with one step per tile, rounded up to a
  // pair of steps (the pair's padding tile past the keys reads as zeros).
  const int n_tiles = uniform(SPT == 2 ? (kv_end + kBN - 1) / kBN : 2 * ((kv_end + 63) / 64));
  if (n_tiles == 0) return;
  const int wave_kv_end = CAUSAL ? min(kv_end, r0 + kRows) : kv_end;
  // 32-key steps of this wave, rounded up to a pair.  A padding step covers
  // keys at or past the wave's range: they are masked (past S or past every
  // row of the wave) and lie in the last staged tile, so they contribute zero.
  const int n_h = uniform(active ? 2 * ((wave_kv_end + 63) / 64) : 0);

  const int h = kvh * p.G + hl;
  const half_t* __restrict__ Qh = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const half_t* __restrict__ Kh = p.k + (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh;
  const half_t* __restrict__ Vh = p.v + (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh;
  half_t* __restrict__ Oh = p.o + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;

  // ---- K/V tile staging through registers: chunk i of this thread is
  // 16-byte chunk tid + 256 i of the K (then V) tile: row st_r[i], global
  // chunk st_c[i], stored at chunk position st_c[i] ^ tswz(row).  Tile j is
  // read through a buffer resource based at its first row whose range ends
  // with row min(64, key_lim - 64 j) - 1: rows past it read as zeros, and the
  // per-lane offsets are loop invariants, so a tile costs no address VALU.
  constexpr int PER_T = kBN * CPR / kPThreads;  // chunks per thread per matrix
  uint4_t kst[PER_T], vst[PER_T];
  int kvo[PER_T], vvo[PER_T];
#pragma unroll
  for (int i = 0; i < PER_T; ++i) {
    const int q = tid + i * kPThreads;
    const int r = q / CPR, cc = q % CPR;
    kvo[i] = (int)(r * p.k_ss * 2) + 16 * cc;
    vvo[i] = (int)(r * p.v_ss * 2) + 16 * cc;
  }
  auto load_tile_to = [&](int j, uint4_t (&kd)[PER_T], uint4_t (&vd)[PER_T]) {
    // Rows of tile j below key_lim; none for a padding tile (an empty range:
    // every read returns zeros and no memory is touched).
    const int rows = uniform(min(kBN, key_lim - j * kBN));
    const int64_t row0 = (int64_t)j * kBN;
    const int kbytes = rows > 0 ? (int)((rows - 1) * p.k_ss * 2) + ROWB : 0;
    const int vbytes = rows > 0 ? (int)((rows - 1) * p.v_ss * 2) + ROWB : 0;
    const auto kr = __builtin_amdgcn_make_buffer_rsrc((void*)(Kh + row0 * p.k_ss), 0, kbytes,
                                                      kBufferWord3);
    const auto vr = __builtin_amdgcn_make_buffer_rsrc((void*)(Vh + row0 * p.v_ss), 0, vbytes,
                                                      kBufferWord3);
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      kd[i] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(kr, kvo[i], 0, 0));
      vd[i] = __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(vr, vvo[i], 0, 0));
    }
  };
  auto load_tile = [&](int j) { load_tile_to(j, kst, vst); };
  auto store_tile_from = [&](int j, const uint4_t (&kd)[PER_T], const uint4_t (&vd)[PER_T]) {
    char* buf = lds + (j % kNBuf) * BUFB;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int q = tid + i * kPThreads;
      const int r = q / CPR, cc = q % CPR;
      const int off = r * ROWB + ((cc ^ tswz<D>(r)) * 16);
      *reinterpret_cast<uint4_t*>(buf + off) = kd[i];
      *reinterpret_cast<uint4_t*>(buf + TILEB + off) = vd[i];
    }
  };
  auto store_tile = [&](int j) { store_tile_from(j, kst, vst); };

  // ---- per-lane LDS byte offsets (within a tile buffer) of the fragments
  // K rows for S^T: key l32 of the step, chunks g * HALF / 8 + s.
  int koff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) koff[s] = l32 * ROWB + (((g * HALF / 8) + s) ^ tswz<D>(l32)) * 16;
  // V^T via tr16: source lane s16 addresses key 4g + s16 / 4 of each 16-key
  // block and dims 32n + 16 * ((lane >> 4) & 1) + 4 * (s16 % 4).  The second
  // 8 keys of a 16-key block sit 8 rows on, where the swizzle differs by 2
  // (voffh); 16 and 32 rows on it repeats.
  const int s16 = lane & 15;
  const int vrow = 4 * g + (s16 >> 2);
  const int vcl = 2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1);
  int voff[NT], voffh[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    voff[n] = TILEB + vrow * ROWB + (((4 * n + vcl) ^ tswz<D>(vrow)) * 16) + (s16 & 1) * 8;
    voffh[n] =
        TILEB + (vrow + 8) * ROWB + (((4 * n + vcl) ^ tswz<D>(vrow + 8)) * 16) + (s16 & 1) * 8;
  }

  // ---- Q^T fragments of the two 32-row blocks: lane -> row, dims g*HALF + 8s + e.
  v8 qf[NRB][KS];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int row = r0 + 32 * rb + l32;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4_t v = {0, 0, 0, 0};
      // Var-len query rows at or past the length are read as zeros: their
      // outputs are unspecified, and non-finite padding is kept out of every
      // computation.
      if (active && row < (VARLEN ? len : S)) v = ld16(Qh + (int64_t)row * p.q_ss + g * HALF + 8 * s);
      // A negative scale is applied as (-Q) K^T times |scale| (sign bits
      // flipped, exact in fp16 and bf16), so every step below sees a positive
      // scale: the running max, the -inf mask and the overflow test keep
      // their meaning.
      if (p.neg_q) v ^= uint4_t{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
      qf[rb][s] = E::as8(v);
    }
  }

  float16_t oacc[NRB][NT];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[rb][n][r] = 0.f;
  float m_run[NRB], l_part[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    m_run[rb] = AKT_P_NEG_INF;
    l_part[rb] = 0.f;
  }
  const float c = p.qk_scale;
  // Per-lane causal / length limit: element r of a step's S^T holds key
  // kh0 + 8 (r / 4) + 4 g + r % 4 of row r0 + 32 rb + l32.
  int lim_base[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int row = r0 + 32 * rb + l32;
    lim_base[rb] = (CAUSAL ? min(row, S - 1) : S - 1) - 4 * g;
  }

  float16_t sA[NRB], sB[NRB];
  uint32_t pA[NRB][8], pB[NRB][8];  // pB starts as P(-1) = 0; pA is written before it is read
  v8 vf[2][NT];                 // V fragments for the next P.V
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int i = 0; i < 8; ++i) pB[rb][i] = 0u;

  // Fragment reads of 32-key step t (its tile must be published).
  auto load_kf = [&](int t, v8 (&kf)[KS]) {
    const char* kb = lds + ((t / SPT) % kNBuf) * BUFB + (t % SPT) * 32 * ROWB;
#pragma unroll
    for (int s = 0; s < KS; ++s) kf[s] = E::as8(*reinterpret_cast<const uint4_t*>(kb + koff[s]));
  };
  auto load_vf = [&](int t, v8 (&vf)[2][NT]) {
    const char* vb = lds + ((t / SPT) % kNBuf) * BUFB + (t % SPT) * 32 * ROWB;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const uint2 lo = ds_read_tr16(vb + voff[n] + u * 16 * ROWB);
        const uint2 hi = ds_read_tr16(vb + voffh[n] + u * 16 * ROWB);
        vf[u][n] = E::as8(uint4_t{lo.x, lo.y, hi.x, hi.y});
      }
  };
  // S^T = K . Q^T for one step.
  auto qk_mfma = [&](const v8 (&kf)[KS], float16_t (&sdst)[NRB]) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sdst[rb][r] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) sdst[rb] = E::mfma(kf[s], qf[rb][s], sdst[rb]);
  };
  // O^T += V^T . P^T for one step.
  auto pv_mfma = [&](const v8 (&vf)[2][NT], const uint32_t (&pk)[NRB][8]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      v8 bop[NRB];
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
        bop[rb] = E::as8(uint4_t{pk[rb][4 * u], pk[rb][4 * u + 1], pk[rb][4 * u + 2],
                                 pk[rb][4 * u + 3]});
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) oacc[rb][n] = E::mfma(vf[u][n], bop[rb], oacc[rb][n]);
    }
  };
  auto qk = [&](int t, float16_t (&sdst)[NRB]) {
    v8 kf[KS];
    load_kf(t, kf);
    qk_mfma(kf, sdst);
  };
  auto pv = [&](int t, const uint32_t (&pk)[NRB][8]) {
    v8 vf[2][NT];
    load_vf(t, vf);
    pv_mfma(vf, pk);
  };
  // Probabilities of S(t) against the running max m_run: P rounded to the
  // operand type into pk and, in l_step, each lane's sum of the 16 rounded
  // probabilities it holds: row l32's keys of lane half g (v_dot2 against ones on the VALU, so
  // every row's sum is its own).  l_part keeps these half-row sums; the two
  // halves are added once, for the output.
  auto softmax = [&](const float16_t (&ss)[NRB], uint32_t (&pk)[NRB][8], float (&l_step)[NRB]) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(__builtin_fmaf(ss[rb][r], c, -m_run[rb]));
        const float p1 = fast_exp2(__builtin_fmaf(ss[rb][r + 1], c, -m_run[rb]));
        pk[rb][r >> 1] = E::pack2(p0, p1);
      }
    }
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ls = E::dot2(pk[rb][i], E::kOnes, ls);
      l_step[rb] = ls;
    }
  };
  // Masks S(t): keys past a row (causal) or past S read -inf.  The tests are
  // wave-uniform and made per 32-row block: only a block whose rows the
  // step's keys reach, or whose keys reach S, runs the selects, and a causal
  // block whose rows all precede the step's first key is set to -inf whole.
  // (With two blocks, the first diagonal step leaves the lower block
  // unmasked and the second masks the upper block whole.)
  auto mask_step = [&](int t, float16_t (&ss)[NRB]) {
    const int kh0 = t * 32;
    if ((CAUSAL && kh0 + 31 > r0) || kh0 + 32 > S) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        if (CAUSAL && kh0 >= r0 + 32 * rb + 32) {
#pragma unroll
          for (int r = 0; r < 16; ++r) ss[rb][r] = AKT_P_NEG_INF;
        } else if ((CAUSAL && kh0 + 31 > r0 + 32 * rb) || kh0 + 32 > S) {
          const int lim = lim_base[rb] - kh0;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) > lim) ss[rb][r] = AKT_P_NEG_INF;
        }
      }
    }
  };
  // Row max of a masked S block in log2 units (IEEE maximum: NaN-propagating,
  // needs no operand canonicalisation).
  auto row_max = [&](const float16_t& sv) {
    float mx = sv[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, sv[r]);
    float a, b;
    swap32(mx, a, b);
    return __builtin_elementwise_maximum(a, b) * c;
  };
  // One pipeline step t < n_h: mask S(t); then, in one scheduling region,
  // the fragment reads, P.V(t-1), S(t+1) and the probabilities of S(t) -- the
  // MFMAs and the softmax VALU work are independent, so the scheduler can
  // interleave them and keep both pipes busy.  The probabilities use the
  // running max as it stands, so no per-step row max is needed: the step's 32
  // probabilities of a row sum to at most 32 * 2^kRescaleSlack unless one of
  // them exceeds 2^kRescaleSlack.  A larger (or NaN) sum takes the rare
  // branch (in step 0, whose row max starts m_run, only for a NaN): the row max is
  // computed, rows whose max exceeds m_run by more than kRescaleSlack (log2
  // units) raise m_run, the normaliser and O are rescaled (after P.V(t-1),
  // computed on the old max, has been accumulated) and the step's
  // probabilities are recomputed.  Otherwise every P stays below
  // 32 * 2^kRescaleSlack, far inside fp16's range.
  auto step = [&](int t, float16_t (&scur)[NRB], float16_t (&snext)[NRB],
                  const uint32_t (&pprev)[NRB][8], uint32_t (&pcur)[NRB][8]) {
    mask_step(t, scur);  // S(0) was masked before the loop too: masking is idempotent
    v8 kf[KS];
    if constexpr (!kPrefetchV) load_vf(t > 0 ? t - 1 : 0, vf);
    load_kf(t + 1, kf);

    pv_mfma(vf, pprev);
    qk_mfma(kf, snext);
    // V of step t, for P.V(t) at the top of step t + 1 (its tile is published).
    if constexpr (kPrefetchV) load_vf(t, vf);

    float l_step[NRB];
    softmax(scur, pcur, l_step);
    // Issue order of the region: each P.V / QK MFMA followed by two VALU
    // instructions, so one wave alternates its matrix and vector work instead
    // of issuing them in clusters.  Two per MFMA, not more: the wave issues in
    // order, and a longer VALU run between MFMAs (three) left the matrix pipe
    // idle at D = 128 (16% slower there, the same at D = 64 and 256).
#pragma unroll
    for (int i = 0; i < (D >= 192 ? 2 * D / 16 : 16); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
    }
    bool over = false;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) over |= !(l_step[rb] <= kStepSumLimit);
    if (__any(over)) {  // wave-uniform, rare
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        const float mx = row_max(scur[rb]);
        const bool raise = mx > m_run[rb] + kRescaleSlack;
        const float alpha = raise ? fast_exp2(m_run[rb] - mx) : 1.f;
        l_part[rb] *= alpha;  // this lane's row
        if (raise) {
          m_run[rb] = mx;
#pragma unroll
          for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[rb][n][r] *= alpha;
        }
      }
      softmax(scur, pcur, l_step);
    }
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) l_part[rb] += l_step[rb];
  };

  // Tiles 0..2 and Q are requested together (one round trip); tiles 0 and 1
  // go to LDS, tile 2 waits in the staging registers.
  {
    uint4_t k0[PER_T], v0[PER_T], k1[PER_T], v1[PER_T];
    load_tile_to(0, k0, v0);
    if (n_tiles > 1) load_tile_to(1, k1, v1);
    if (n_tiles > 2) load_tile(2);
    store_tile_from(0, k0, v0);
    if (n_tiles > 1) store_tile_from(1, k1, v1);
  }
  __syncthreads();
  // S(0) (tile 0 is always staged), masked; its row max starts the running
  // max, so step 0's probabilities are at most 1 and its sums never take the
  // raise branch.  Every row has a valid key in step 0 (key 0: causal rows
  // are >= 0 and S >= 1), so the start is finite for finite inputs.
  qk(0, sA);
  if constexpr (kPrefetchV) load_vf(0, vf);  // P.V(-1) of step 0 multiplies P = 0
  mask_step(0, sA);
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) m_run[rb] = row_max(sA[rb]);
  // Publishes tile j + 1 (stored before the previous barrier) and retires the
  // buffer of tile j - 2, which now takes tile j + 2 from the staging
  // registers; tile j + 3 is then fetched into them.  Step t reads K of step
  // t + 1 and V of step t - 1, so a step's turn comes at its own tile.
  auto tile_turn = [&](int j) {
    __syncthreads();
    if (j + 2 < n_tiles) store_tile(j + 2);
    if (j + 3 < n_tiles) load_tile(j + 3);
  };
  // Steps run in pairs (t, t + 1) (one tile of two steps, or two tiles of one
  // step); n_h is even.  At the top of a pair: sA = S(t) and pB = P(t - 1)
  // (zero for t = 0).  The last pair's S(t + 2) is computed from whatever its
  // buffer holds and never used; the pair is followed by the drain P.V(t + 1).
#pragma clang loop unroll(disable)
  for (int j = 0; j < n_tiles; j += 2 / SPT) {
    tile_turn(j);
    const int t = SPT * j;
    if (t < n_h) step(t, sA, sB, pB, pA);  // wave-uniform
    if constexpr (SPT == 1) tile_turn(j + 1);  // n_tiles is even
    if (t < n_h) {
      step(t + 1, sB, sA, pA, pB);
      if (t + 2 == n_h) {  // drain: P.V(n_h - 1)
        if constexpr (kPrefetchV) pv_mfma(vf, pB);
        else pv(t + 1, pB);
      }
    }
  }

  // ---- epilogue: O is normalised, transposed through LDS and written as
  // whole rows.  Each lane holds 4-element pieces of one row, so writing them
  // straight to HBM costs one store instruction per piece, each spread over
  // 32 rows; through LDS every lane stores 16 contiguous bytes and a wave
  // stores whole rows.  The barrier retires every tile buffer first (all
  // waves pass it: the loop's turn count is the workgroup's).
  __syncthreads();
  if (!active) return;
  // The row index is derived again here (the opaque copy keeps the compiler
  // from holding the prologue's row registers live through the loop).
  int lane_e = lane;
  asm volatile("" : "+v"(lane_e));
  static_assert(kSlots * kRows * ROWB <= kNBuf * BUFB, "O staging fits the tile buffers");
  char* ost = lds + wave * (kRows * ROWB);  // this wave's rows, 16-byte chunks swizzled
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int lr = 32 * rb + (lane_e & 31);  // row within the wave's block
    const int row = r0 + lr;
    // Row l32's normaliser sits in lane l32 (rows 0..15) or l32 + 16.
    const float l_row = xor32_sum(l_part[rb]);  // both key halves of row l32
    const float inv = l_row > 0.f ? __builtin_amdgcn_rcpf(l_row) : 0.f;
    if (p.lse && g == 0 && row < row_lim) {
      // ln sum_k exp(scale * q.k) = (m + log2 l) * ln 2: P = exp2(c s - m) and
      // l sums the fp16-rounded P (the reference's commented-out store at
      // prefill_flash_attention.py:331-333 is m + log l in natural units).
      p.lse[(int64_t)b * p.lse_sb + (int64_t)h * p.lse_sh + (int64_t)row * p.lse_ss] =
          l_row > 0.f ? (m_run[rb] + __log2f(l_row)) * kLn2 : AKT_P_NEG_INF;
    }
    // Element r of oacc[rb][n] is dim 32 n + 8 (r / 4) + 4 g + r % 4: half of
    // 16-byte chunk 4 n + r / 4.
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float16_t& a = oacc[rb][n];
        const uint2 hv = {E::pack2(a[4 * q4] * inv, a[4 * q4 + 1] * inv),
                          E::pack2(a[4 * q4 + 2] * inv, a[4 * q4 + 3] * inv)};
        const int chunk = (4 * n + q4) ^ eswz(lr);
        *reinterpret_cast<uint2*>(ost + lr * ROWB + chunk * 16 + 8 * g) = hv;
      }
  }
  // Row-major read back: lane i takes chunk i % CPR of row i / CPR (+ 64 / CPR
  // rows per pass); the LDS writes above are this wave's own and complete in order.
#pragma unroll
  for (int idx = lane_e; idx < kRows * CPR; idx += 64) {
    const int lr = idx / CPR, cc = idx % CPR;
    const uint4_t v = *reinterpret_cast<const uint4_t*>(ost + lr * ROWB + ((cc ^ eswz(lr)) * 16));
    const int row = r0 + lr;
    if (row < row_lim) *reinterpret_cast<uint4_t*>(Oh + (int64_t)row * p.o_ss + 8 * cc) = v;
  }
}

template <int D, bool CAUSAL, bool VARLEN, bool BF16, bool LONG>
int launch(const PrefillParams& p, dim3 grid, hipStream_t st) {
  KernelTimer timer;
  timer.launch(prefill_kernel<D, CAUSAL, VARLEN, BF16, LONG>, grid, dim3(kPThreads), 0, st, p);
  return check_launch("prefill_kernel");
}

template <int D, bool BF16, bool LONG>
int launch_dt(bool causal, bool varlen, const PrefillParams& p, dim3 grid, hipStream_t st) {
  if (causal)
    return varlen ? launch<D, true, true, BF16, LONG>(p, grid, st)
                  : launch<D, true, false, BF16, LONG>(p, grid, st);
  return varlen ? launch<D, false, true, BF16, LONG>(p, grid, st)
                : launch<D, false, false, BF16, LONG>(p, grid, st);
}

template <int D, bool LONG>
int launch_l(bool bf16, bool causal, bool varlen, const PrefillParams& p, dim3 grid,
             hipStream_t st) {
  return bf16 ? launch_dt<D, true, LONG>(causal, varlen, p, grid, st)
              : launch_dt<D, false, LONG>(causal, varlen, p, grid, st);
}

// long_rows selects the long-sequence instance (D = 128 only).
template <int D>
int launch_d(bool bf16, bool causal, bool varlen, bool long_rows, const PrefillParams& p,
             dim3 grid, hipStream_t st) {
  if constexpr (D == 128) {
    if (long_rows) return launch_l<D, true>(bf16, causal, varlen, p, grid, st);
  }
  return launch_l<D, false>(bf16, causal, varlen, p, grid, st);
}

}  // namespace

// Head dims 192 and 256 are instantiated in a second translation unit of this
// file (prefill_wide.hip, AKT_PREFILL_WIDE_TU), which the build compiles with
// LLVM's iterative ILP machine scheduler: 8-12% faster at those head dims, and
// 1-2% slower at D = 64, so D = 64 and 128 stay here with the default one.
int prefill_launch_wide(int head_dim, bool bf16, bool causal, bool varlen, const PrefillParams& p,
                        dim3 grid, hipStream_t st);
#ifdef AKT_PREFILL_WIDE_TU
int prefill_launch_wide(int head_dim, bool bf16, bool causal, bool varlen, const PrefillParams& p,
                        dim3 grid, hipStream_t st) {
  return head_dim == 192 ? launch_d<192>(bf16, causal, varlen, false, p, grid, st)
                         : launch_d<256>(bf16, causal, varlen, false, p, grid, st);
}
#endif

}  // namespace akt

#ifndef AKT_PREFILL_WIDE_TU
using namespace akt;

namespace {
int prefill_impl(const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch,
                 int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                 const int64_t q_stride[4], const int64_t k_stride[4], const int64_t v_stride[4],
                 const int64_t o_stride[4], const int64_t* lse_stride, float softmax_scale,
                 int causal, const void* varlen, int varlen_bits, int dtype, void* stream) {
  clear_error();
  AKT_CHECK(dtype == AKT_DTYPE_F16 || dtype == AKT_DTYPE_BF16,
            "prefill dtype must be AKT_DTYPE_F16 or AKT_DTYPE_BF16, got %d", dtype);
  AKT_CHECK(batch >= 0 && num_q_heads > 0 && num_kv_heads > 0, "batch/head counts must be positive");
  AKT_CHECK(num_q_heads % num_kv_heads == 0,
            "num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)", (long long)num_q_heads,
            (long long)num_kv_heads);
  if (head_dim != 64 && head_dim != 128 && head_dim != 192 && head_dim != 256)
    return set_error(AKT_ERR_UNSUPPORTED,
                     "prefill head_dim %lld not supported (64, 128, 192, 256)",
                     (long long)head_dim);
  AKT_CHECK(seq_len >= 0 && seq_len < (1ll << 30), "seq_len out of range");
  AKT_CHECK(q_stride[3] == 1 && k_stride[3] == 1 && v_stride[3] == 1 && o_stride[3] == 1,
            "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(q, q_stride, 3) && rows_aligned16(k, k_stride, 3) &&
                rows_aligned16(v, v_stride, 3) && rows_aligned16(o, o_stride, 3),
            "tensors must have 16-byte aligned rows");
  AKT_CHECK(!varlen || varlen_bits == 32 || varlen_bits == 64, "varlen_bits must be 32 or 64");
  AKT_CHECK(std::isfinite(softmax_scale), "softmax_scale must be finite");
  AKT_CHECK(!lse || (lse_stride && aligned4(lse)), "lse needs strides and 4-byte alignment");
  // K / V tiles are read through 32-bit buffer offsets of up to 64 rows.
  AKT_CHECK(k_stride[2] >= 0 && k_stride[2] < (1 << 22) && v_stride[2] >= 0 &&
                v_stride[2] < (1 << 22),
            "K / V sequence stride out of range [0, 2^22)");
  if (batch == 0 || seq_len == 0) return AKT_OK;

  PrefillParams p = {};
  p.q = (const half_t*)q;
  p.k = (const half_t*)k;
  p.v = (const half_t*)v;
  p.o = (half_t*)o;
  p.varlen = varlen;
  p.varlen_bits = varlen_bits;
  p.lse = lse;
  if (lse) {
    p.lse_sb = lse_stride[0];
    p.lse_sh = lse_stride[1];
    p.lse_ss = lse_stride[2];
  }
  p.q_sb = q_stride[0]; p.q_sh = q_stride[1]; p.q_ss = q_stride[2];
  p.k_sb = k_stride[0]; p.k_sh = k_stride[1]; p.k_ss = k_stride[2];
  p.v_sb = v_stride[0]; p.v_sh = v_stride[1]; p.v_ss = v_stride[2];
  p.o_sb = o_stride[0]; p.o_sh = o_stride[1]; p.o_ss = o_stride[2];
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.S = (int)seq_len;
  const bool long_rows = head_dim == 128 && seq_len >= kLongRowsD128;
  p.n_rb = (int)ceil_div(seq_len, rows_for((int)head_dim, long_rows));
  p.n_sg = (int)ceil_div((int64_t)p.G * p.n_rb, kSlots);
  p.grid1d = (batch > 65535 || p.n_sg > 65535) ? 1 : 0;
  p.fast_div = ((int64_t)p.G * p.n_rb + kSlots < (1ll << 22)) ? 1 : 0;
  p.g_inv = 1.0f / (float)p.G;
  // Any finite scale: a negative one flips Q's sign in the kernel; a zero (or
  // subnormal) one becomes FLT_MIN, whose product with any score below 2^100
  // in magnitude lies within 2^-25 of 0, so every visible key gets probability
  // exp2(0) = 1, which is softmax at scale 0, while masked keys (-inf) still
  // get 0.
  p.neg_q = softmax_scale < 0.f ? 1 : 0;
  p.qk_scale = fmaxf(fabsf(softmax_scale) * kLog2e, FLT_MIN);
  const int64_t n_wg = batch * num_kv_heads * p.n_sg;
  AKT_CHECK(n_wg < (1ll << 31), "problem too large");
  const dim3 grid = p.grid1d ? dim3((unsigned)n_wg)
                             : dim3((unsigned)num_kv_heads, (unsigned)batch, (unsigned)p.n_sg);
  const bool is_causal = causal != 0;
  const bool is_var = varlen != nullptr;
  hipStream_t st = (hipStream_t)stream;
  const bool bf16 = dtype == AKT_DTYPE_BF16;
  if (head_dim == 64) return launch_d<64>(bf16, is_causal, is_var, false, p, grid, st);
  if (head_dim == 128) return launch_d<128>(bf16, is_causal, is_var, long_rows, p, grid, st);
  return prefill_launch_wide((int)head_dim, bf16, is_causal, is_var, p, grid, st);
}
}  // namespace

extern "C" int akt_prefill_fwd(const void* q, const void* k, const void* v, void* o, int64_t batch,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                               int64_t head_dim, const int64_t q_stride[4],
                               const int64_t k_stride[4], const int64_t v_stride[4],
                               const int64_t o_stride[4], float softmax_scale, int causal,
                               const void* varlen, int varlen_bits, void* stream) {
  return prefill_impl(q, k, v, o, nullptr, batch, num_q_heads, num_kv_heads, seq_len, head_dim,
                      q_stride, k_stride, v_stride, o_stride, nullptr, softmax_scale, causal,
                      varlen, varlen_bits, AKT_DTYPE_F16, stream);
}

extern "C" int akt_prefill_fwd_lse(const void* q, const void* k, const void* v, void* o,
                                   float* lse, int64_t batch, int64_t num_q_heads,
                                   int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                   const int64_t q_stride[4], const int64_t k_stride[4],
                                   const int64_t v_stride[4], const int64_t o_stride[4],
                                   const int64_t lse_stride[3], float softmax_scale, int causal,
                                   const void* varlen, int varlen_bits, void* stream) {
  if (!lse) {
    clear_error();
    return set_error(AKT_ERR_INVALID_ARGUMENT, "lse output pointer is required");
  }
  return prefill_impl(q, k, v, o, lse, batch, num_q_heads, num_kv_heads, seq_len, head_dim,
                      q_stride, k_stride, v_stride, o_stride, lse_stride, softmax_scale, causal,
                      varlen, varlen_bits, AKT_DTYPE_F16, stream);
}

extern "C" int akt_prefill_fwd_ex(const void* q, const void* k, const void* v, void* o,
                                  float* lse, int64_t batch, int64_t num_q_heads,
                                  int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                  const int64_t q_stride[4], const int64_t k_stride[4],
                                  const int64_t v_stride[4], const int64_t o_stride[4],
                                  const int64_t lse_stride[3], float softmax_scale, int causal,
                                  const void* varlen, int varlen_bits, int dtype, void* stream) {
  return prefill_impl(q, k, v, o, lse, batch, num_q_heads, num_kv_heads, seq_len, head_dim,
                      q_stride, k_stride, v_stride, o_stride, lse ? lse_stride : nullptr,
                      softmax_scale, causal, varlen, varlen_bits, dtype, stream);
}
#endif  // AKT_PREFILL_WIDE_TU
