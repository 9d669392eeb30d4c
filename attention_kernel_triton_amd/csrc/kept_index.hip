// Kept-token index selection on the GPU.
//
// The reference builds the sparse-decode index lists in host-driven torch code
// (sparsetoken_decode_flash_attention_redundant.py:283-295,
//  sparsetoken_decode_flash_attention_redundant_var_len_paged.py:341-353,
//  magicpig_..._with_norm.py:327-338): keep = rand(n) < p; if nothing is kept,
// keep index 0; indices = nonzero(keep) ascending; pad with -1; nnz = count.
// This kernel produces the same int32 arrays in one launch, one workgroup per
// row.  A step covers 32768 elements: thread t of 1024 owns 32 consecutive ones
// (a whole row of typical length is one step, with all its loads in flight), so
// its kept elements are ranked by a popcount of its 32-bit keep mask plus an
// exclusive prefix over the workgroup's threads (a wave scan, then the 16
// wave totals through LDS), and the loads of step s + 1 are in flight while
// step s is ranked.  The loads go through a buffer resource that ends at the
// row's last element, so nothing past the row is read.
#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kKThreads = 1024;
constexpr int kKWaves = kKThreads / kWave;
constexpr int kPer = 32;                 // elements per thread per step
constexpr int kStep = kKThreads * kPer;  // elements per step

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int u = __shfl_up(v, d, kWave);
    v += lane >= d ? u : 0;
  }
  return v;
}

template <bool FROM_MASK>
__global__ __launch_bounds__(kKThreads) void kept_index_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ uniform, float ratio, int64_t n,
    int64_t row_stride, const int32_t* __restrict__ row_len, int32_t* __restrict__ ind,
    int64_t l_max, int32_t* __restrict__ nnz, int ensure_nonempty) {
  __shared__ int wave_tot[2][kKWaves];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int64_t nr = n;
  if (row_len) {
    const int64_t v = row_len[r];
    nr = v < 0 ? 0 : (v > n ? n : v);
  }
  int32_t* out = ind + (int64_t)r * l_max;
  // The row's elements [0, nr) (row lengths below 2^28: byte offsets fit 31 bits).
  const int esz = FROM_MASK ? 1 : 4;
  const void* row_base = FROM_MASK ? (const void*)(mask + (int64_t)r * row_stride)
                                   : (const void*)(uniform + (int64_t)r * row_stride);
  const auto rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)row_base, 0, (int)(nr * esz),
                                                      kBufferWord3);
  // This thread's kPer elements of a step as raw words (fp32 draws: one word
  // each; mask bytes: four to a word).
  constexpr int NW = FROM_MASK ? kPer / 4 : kPer;
  auto load = [&](int64_t base, uint32_t (&w)[NW]) {
    const int off = (int)((base + (int64_t)kPer * tid) * esz);
    if constexpr (FROM_MASK) {
      // Byte loads: a mask row need not start 4-byte aligned.
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        uint32_t x = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          x |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rsrc, off + 4 * i + k, 0, 0) << (8 * k);
        w[i] = x;
      }
    } else {
#pragma unroll
      for (int i = 0; i < NW / 4; ++i) {
        const uint4_t v = __builtin_bit_cast(
            uint4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 16 * i, 0, 0));
        w[4 * i] = v[0];
        w[4 * i + 1] = v[1];
        w[4 * i + 2] = v[2];
        w[4 * i + 3] = v[3];
      }
    }
  };
  uint32_t cur[NW], nxt[NW];
  if (nr > 0) load(0, cur);
  int count = 0;  // kept so far (uniform across the workgroup)
  int buf = 0;
  for (int64_t base = 0; base < nr; base += kStep) {
    if (base + kStep < nr) load(base + kStep, nxt);
    // Keep mask of this thread's elements (bit i: element base + kPer tid + i).
    const int64_t j0 = base + (int64_t)kPer * tid;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      bool keep;
      if constexpr (FROM_MASK) keep = ((cur[i >> 2] >> (8 * (i & 3))) & 0xffu) != 0;
      else keep = __builtin_bit_cast(float, cur[i]) < ratio;
      m |= (keep && j0 + i < nr) ? (1u << i) : 0u;
    }
    const int c = __builtin_popcount(m);
    const int incl = wave_inclusive_scan(c, lane);
    if (lane == kWave - 1) wave_tot[buf][wave] = incl;
    __syncthreads();
    int before = incl - c, step_total = 0;
#pragma unroll
    for (int w = 0; w < kKWaves; ++w) {
      const int t = wave_tot[buf][w];
      before += (w < wave) ? t : 0;
      step_total += t;
    }
    int64_t slot = (int64_t)count + before;
    while (m) {
      const int i = __builtin_ctz(m);
      m &= m - 1;
      if (slot < l_max) out[slot] = (int32_t)(j0 + i);
      ++slot;
    }
    count += step_total;
    buf ^= 1;  // the other buffer is free: every wave read it before this step's barrier
#pragma unroll
    for (int i = 0; i < NW; ++i) cur[i] = nxt[i];
  }
  int total = count;
  if (total == 0 && ensure_nonempty) {
    if (tid == 0 && l_max > 0) out[0] = 0;
    total = 1;
  }
  for (int64_t i = (int64_t)total + tid; i < l_max; i += kKThreads) out[i] = -1;
  if (tid == 0) nnz[r] = total;
}

int launch_kept(bool from_mask, const uint8_t* mask, const float* uniform, float ratio,
                int64_t rows, int64_t n, int64_t row_stride, const int32_t* row_len,
                int32_t* sparse_ind, int64_t l_max, int32_t* sparse_nnz, int ensure_nonempty,
                void* stream) {
  clear_error();
  AKT_CHECK(rows >= 0 && rows < (1ll << 31) && n >= 0 && l_max >= 0, "sizes out of range");
  AKT_CHECK(row_stride >= n, "row stride (%lld) smaller than row length (%lld)",
            (long long)row_stride, (long long)n);
  AKT_CHECK(n < (1ll << 28), "row length (%lld) must be below 2^28", (long long)n);
  AKT_CHECK(sparse_nnz && (sparse_ind || l_max == 0), "output pointers are required");
  if (rows == 0) return AKT_OK;
  AKT_CHECK(from_mask ? (mask || n == 0) : (uniform || n == 0), "input pointer is required");
  hipStream_t st = (hipStream_t)stream;
  KernelTimer timer;
  if (from_mask) {
    timer.launch(kept_index_kernel<true>, dim3((unsigned)rows), dim3(kKThreads), 0, st, mask,
                 (const float*)nullptr, 0.f, n, row_stride, row_len, sparse_ind, l_max,
                 sparse_nnz, ensure_nonempty);
  } else {
    timer.launch(kept_index_kernel<false>, dim3((unsigned)rows), dim3(kKThreads), 0, st,
                 (const uint8_t*)nullptr, uniform, ratio, n, row_stride, row_len, sparse_ind,
                 l_max, sparse_nnz, ensure_nonempty);
  }
  return check_launch("kept_index_kernel");
}

}  // namespace
}  // namespace akt

extern "C" int akt_kept_index_from_mask(const uint8_t* mask, int64_t rows, int64_t n,
                                        int64_t mask_row_stride, const int32_t* row_len,
                                        int32_t* sparse_ind, int64_t l_max, int32_t* sparse_nnz,
                                        int ensure_nonempty, void* stream) {
  return akt::launch_kept(true, mask, nullptr, 0.f, rows, n, mask_row_stride, row_len, sparse_ind,
                          l_max, sparse_nnz, ensure_nonempty, stream);
}

extern "C" int akt_kept_index_from_uniform(const float* uniform, float kept_ratio, int64_t rows,
                                           int64_t n, int64_t row_stride, const int32_t* row_len,
                                           int32_t* sparse_ind, int64_t l_max,
                                           int32_t* sparse_nnz, int ensure_nonempty,
                                           void* stream) {
  return akt::launch_kept(false, nullptr, uniform, kept_ratio, rows, n, row_stride, row_len,
                          sparse_ind, l_max, sparse_nnz, ensure_nonempty, stream);
}
