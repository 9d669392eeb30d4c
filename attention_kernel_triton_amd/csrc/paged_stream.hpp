// Stream-K paged decode (paged_stream.hip): parameters and host entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "akt_common.hpp"

namespace akt {

// Largest batch whose sequence table fits the kernel's LDS.
constexpr int kStreamMaxBatch = 1024;
// Most waves a launch uses.  A wave stores its partial of unit u at slot
// wave + u, so a launch needs (its waves + units) partial slots.
constexpr int kStreamMaxWaves = 4096;

struct StreamParams {
  const half_t* q;      // [B, Hq, D] rows (strides q_sb, q_sh)
  const half_t* kbase;  // KV pool, K half
  const half_t* vbase;  // KV pool + the K/V axis stride
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  half_t* o;      // [B, Hq, D] contiguous
  float* lse;     // [B, Hq] or null
  int* arrive;    // [B * Y] arrival counters (zero between launches)
  float* part_o;  // [waves + B * Y, GT, D]
  float* part_ml; // [waves + B * Y, GT, 4]: max, fp16-P normaliser, fp32 normaliser, pad
  int64_t q_sb, q_sh;
  int64_t k_sa, k_head, v_sa, v_head;  // page and kv-head strides (elements)
  int k_sb, v_sb;                      // row strides (elements, < 2^26)
  int B, Hq, G, Y, n_hg;
  int page_size, gpp;  // gpp = page_size / 16 groups per page
  int total_pages;
  int TG;              // groups per head group: total_pages * gpp
  int N;               // groups of the launch: Y * TG (< 2^31)
  int W;               // waves of the launch (set by paged_stream_launch)
  int num_pool_pages;
  float qk_scale;      // softmax_scale * log2(e)
};

// Whether a paged decode can take the stream-K kernel: pages of whole
// 16-token groups, a batch that fits the LDS table and a group axis that fits
// 32 bits.
bool paged_stream_eligible(int64_t batch, int64_t page_size, int64_t total_pages, int64_t Y);

// Waves a launch of instance (D, gt) uses at most on the current device
// (resident workgroups x 4, at most kStreamMaxWaves; kStreamMaxWaves when the
// device cannot be queried).
int64_t paged_stream_wave_cap(int D, int gt);

// Launches the kernel for head dim D with gt heads per unit; p.W is set here.
int paged_stream_launch(StreamParams p, int D, int gt, hipStream_t st);

}  // namespace akt
