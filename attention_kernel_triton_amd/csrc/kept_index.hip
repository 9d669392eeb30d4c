// Kept-token index selection on the GPU.
//
// The reference builds the sparse-decode index lists in host-driven torch code
// (sparsetoken_decode_flash_attention_redundant.py:283-295,
//  sparsetoken_decode_flash_attention_redundant_var_len_paged.py:341-353,
//  magicpig_..._with_norm.py:327-338): keep = rand(n) < p; if nothing is kept,
// keep index 0; indices = nonzero(keep) ascending; pad with -1; nnz = count.
// This kernel produces the same int32 arrays in one launch: one workgroup per
// row scans the row in 256-element steps, ranks kept elements with wave
// ballots plus an LDS prefix over the four waves, and writes them in order.
#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kKThreads = 256;

template <bool FROM_MASK>
__global__ __launch_bounds__(kKThreads) void kept_index_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ uniform, float ratio, int64_t n,
    int64_t row_stride, const int32_t* __restrict__ row_len, int32_t* __restrict__ ind,
    int64_t l_max, int32_t* __restrict__ nnz, int ensure_nonempty) {
  __shared__ int wave_cnt[kKThreads / kWave];
  __shared__ int total_sh;
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
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int count = 0;  // kept so far (uniform across the workgroup)
  for (int64_t base = 0; base < nr; base += kKThreads) {
    const int64_t j = base + tid;
    bool keep = false;
    if (j < nr) {
      if constexpr (FROM_MASK) keep = mask[(int64_t)r * row_stride + j] != 0;
      else keep = uniform[(int64_t)r * row_stride + j] < ratio;
    }
    const uint64_t bal = __ballot(keep);
    if (lane == 0) wave_cnt[wave] = __builtin_popcountll(bal);
    __syncthreads();
    int before = 0, step_total = 0;
#pragma unroll
    for (int w = 0; w < kKThreads / kWave; ++w) {
      const int cw = wave_cnt[w];
      before += (w < wave) ? cw : 0;
      step_total += cw;
    }
    if (keep) {
      const int64_t slot = (int64_t)count + before + __builtin_popcountll(bal & lt_mask);
      if (slot < l_max) out[slot] = (int32_t)j;
    }
    count += step_total;
    __syncthreads();
  }
  if (tid == 0) total_sh = count;
  __syncthreads();
  int total = total_sh;
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
