// Paged KV cache write side: append new K/V tokens into the page pool.
//
// The reference only reads paged caches; its tests build the page tables by
// hand (decode_flash_attention_redundant_var_len_paged.py:349-353,
// sparsetoken_decode_flash_attention_redundant_var_len_paged.py:321-330).
// This is the step that fills them: sequence b's n_b new tokens (rows
// append_indptr[b] .. append_indptr[b+1] of k_new / v_new) are the LAST n_b
// logical positions of b under the (already updated) page table, i.e.
// positions len_b - n_b .. len_b - 1 with
//   len_b = (indptr[b+1] - indptr[b] - 1) * page_size + last_page_len[b].
// Position t lives in page indices[indptr[b] + t / page_size], slot
// t % page_size -- the same addressing the decode kernels read with.
// Tokens whose position or page id falls outside the table / pool are
// skipped, never written.
//
// Work: one wave per run of kTPW consecutive new tokens.  The wave finds the
// sequence of each of its tokens with one ballot per 64 sequences over
// append_indptr (the sequences are consecutive runs of rows), lane t looks
// up token t's page and slot (two rounds of loads for all tokens at once),
// and the lanes then move 16-byte chunks of the tokens' (kv head, dim) rows,
// the loads of token t + 1 issued before the stores of token t.  Each lane
// owns chunks lane + 64 j (j < NPL) of a token's Hkv * D / 8 chunks of K
// (and the same chunks of V); rows of more chunks take several passes.
// HBM-bound: 4 * D bytes per (token, kv head) (read K and V, write K and V).
#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kAThreads = 256;
constexpr int kAWaves = kAThreads / 64;
constexpr int kTPW = 2;  // new tokens per wave (2: 54.5 us on the bench leg; 4: 55.3, 8: 56.6, 16: 63.4)

struct AppendParams {
  const half_t* k_new;
  const half_t* v_new;
  const int32_t* append_indptr;
  half_t* pool;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  int64_t kn_st, kn_sh, vn_st, vn_sh;  // new rows: token / head strides
  int64_t sp, skv, sh, ss;             // pool strides: page, K/V, head, slot
  int64_t total_new;
  int B, Hkv, cpr, page_size, num_pool_pages;
};

template <int NPL>
__global__ __launch_bounds__(kAThreads) void paged_append_kernel(AppendParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int64_t tok0 = ((int64_t)blockIdx.x * kAWaves + wave) * kTPW;
  if (tok0 >= p.total_new) return;  // wave-uniform
  const int nt = (int)min((int64_t)kTPW, p.total_new - tok0);
  const int per_tok = p.Hkv * p.cpr;  // chunks of one token's K (or V) rows

  // Sequence of token tok0 + t: cnt[t] - 1, where cnt[t] counts the
  // sequences b < B with append_indptr[b] <= tok0 + t (the rows of sequence
  // b are append_indptr[b] .. append_indptr[b + 1] - 1).
  int cnt[kTPW];
#pragma unroll
  for (int t = 0; t < kTPW; ++t) cnt[t] = 0;
  for (int jb = 0; jb < p.B; jb += 64) {  // wave-uniform
    const int j = jb + lane;
    const int64_t aj = j < p.B ? (int64_t)p.append_indptr[j] : INT64_MAX;
#pragma unroll
    for (int t = 0; t < kTPW; ++t) cnt[t] += __popcll(__ballot(aj <= tok0 + t));
  }
  // Lane t < nt: token tok0 + t's page id and slot, or page -1 (skipped):
  // the token's rows are the last ones of its sequence under the updated
  // table, positions len - n .. len - 1.
  int my_b = -1;
#pragma unroll
  for (int t = 0; t < kTPW; ++t)
    if (lane == t) my_b = cnt[t] - 1;
  int page = -1, slot = 0;
  if (lane < nt && my_b >= 0) {
    const int64_t tok = tok0 + lane;
    const int64_t a0 = p.append_indptr[my_b], a1 = p.append_indptr[my_b + 1];
    const int ip0 = p.indptr[my_b], ip1 = p.indptr[my_b + 1];
    const int np = ip1 - ip0;
    const int last = min(max(p.last_len[my_b], 0), p.page_size);
    const int64_t len = (int64_t)(np - 1) * p.page_size + last;
    const int64_t pos = len - (a1 - a0) + (tok - a0);
    // A malformed indptr (the token outside its sequence's rows) or a
    // position outside the table writes nothing.
    if (tok >= a0 && tok < a1 && np > 0 && pos >= 0 && pos < len) {
      const int lp = (int)(pos / p.page_size);
      const int pg = p.indices[ip0 + lp];
      if (pg >= 0 && pg < p.num_pool_pages) {
        page = pg;
        slot = (int)(pos - (int64_t)lp * p.page_size);
      }
    }
  }

  // This lane's chunks: (kv head, 16-byte chunk) of chunk index lane + 64 j.
  for (int cb = 0; cb < per_tok; cb += 64 * NPL) {  // wave-uniform passes
    int64_t ksrc[NPL], vsrc[NPL], dst_off[NPL];
    bool has[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = cb + lane + 64 * j;
      has[j] = i < per_tok;
      const int h = has[j] ? i / p.cpr : 0;
      const int c = has[j] ? i - h * p.cpr : 0;
      ksrc[j] = (int64_t)h * p.kn_sh + 8 * c;
      vsrc[j] = (int64_t)h * p.vn_sh + 8 * c;
      dst_off[j] = (int64_t)h * p.sh + 8 * c;
    }
    uint4_t kb[2][NPL], vb[2][NPL];
    // Rows of token tok0 + t; t past the wave's last token re-reads it.
    auto load = [&](int t, uint4_t (&kd)[NPL], uint4_t (&vd)[NPL]) {
      const int64_t tok = tok0 + min(t, nt - 1);
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        kd[j] = has[j] ? ld16(p.k_new + tok * p.kn_st + ksrc[j]) : uint4_t{0, 0, 0, 0};
        vd[j] = has[j] ? ld16(p.v_new + tok * p.vn_st + vsrc[j]) : uint4_t{0, 0, 0, 0};
      }
    };
    load(0, kb[0], vb[0]);
#pragma unroll
    for (int t = 0; t < kTPW; ++t) {
      if (t + 1 < kTPW) load(t + 1, kb[(t + 1) & 1], vb[(t + 1) & 1]);
      const int pg = __builtin_amdgcn_readlane(page, t);
      const int sl = __builtin_amdgcn_readlane(slot, t);
      if (t < nt && pg >= 0) {  // wave-uniform
        half_t* dst = p.pool + (int64_t)pg * p.sp + (int64_t)sl * p.ss;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
          if (has[j]) {
            st16(dst + dst_off[j], kb[t & 1][j]);
            st16(dst + p.skv + dst_off[j], vb[t & 1][j]);
          }
      }
    }
  }
}

}  // namespace
}  // namespace akt

using namespace akt;

extern "C" int akt_paged_kv_append(const void* k_new, const void* v_new,
                                   const int32_t* append_indptr, void* kv_cache,
                                   const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                   const int32_t* kv_last_page_len, int64_t batch,
                                   int64_t total_new, int64_t num_kv_heads, int64_t head_dim,
                                   int64_t page_size, int64_t num_pool_pages,
                                   const int64_t k_new_stride[3], const int64_t v_new_stride[3],
                                   const int64_t kv_stride[5], void* stream) {
  clear_error();
  AKT_CHECK(batch >= 0 && total_new >= 0 && num_kv_heads > 0, "sizes must be non-negative");
  AKT_CHECK(head_dim > 0 && head_dim % 8 == 0 && head_dim <= 1024,
            "head_dim must be a positive multiple of 8 up to 1024");
  AKT_CHECK(page_size > 0 && page_size < (1 << 20), "page_size out of range");
  AKT_CHECK(num_pool_pages >= 0, "num_pool_pages out of range");
  if (batch == 0 || total_new == 0) return AKT_OK;
  AKT_CHECK(k_new && v_new && append_indptr && kv_cache && kv_page_indptr && kv_page_indices &&
                kv_last_page_len && k_new_stride && v_new_stride && kv_stride,
            "all pointers are required");
  AKT_CHECK(k_new_stride[2] == 1 && v_new_stride[2] == 1 && kv_stride[4] == 1,
            "head_dim stride must be 1");
  AKT_CHECK(rows_aligned16(k_new, k_new_stride, 2) && rows_aligned16(v_new, v_new_stride, 2) &&
                rows_aligned16(kv_cache, kv_stride, 4),
            "tensors must have 16-byte aligned rows");
  AppendParams p = {};
  p.k_new = (const half_t*)k_new;
  p.v_new = (const half_t*)v_new;
  p.append_indptr = append_indptr;
  p.pool = (half_t*)kv_cache;
  p.indptr = kv_page_indptr;
  p.indices = kv_page_indices;
  p.last_len = kv_last_page_len;
  p.kn_st = k_new_stride[0];
  p.kn_sh = k_new_stride[1];
  p.vn_st = v_new_stride[0];
  p.vn_sh = v_new_stride[1];
  p.sp = kv_stride[0];
  p.skv = kv_stride[1];
  p.sh = kv_stride[2];
  p.ss = kv_stride[3];
  p.total_new = total_new;
  p.B = (int)batch;
  p.Hkv = (int)num_kv_heads;
  p.cpr = (int)(head_dim / 8);
  p.page_size = (int)page_size;
  p.num_pool_pages = (int)(num_pool_pages < (1ll << 31) ? num_pool_pages : (1ll << 31) - 1);
  AKT_CHECK(num_kv_heads * p.cpr < (1ll << 30), "num_kv_heads * head_dim too large");
  AKT_CHECK(batch < (1ll << 30), "batch too large");  // the kernel steps sequences by 64 in int
  const int64_t grid = ceil_div(ceil_div(total_new, kTPW), kAWaves);
  AKT_CHECK(grid < (1ll << 31), "too many tokens");
  // Chunks per lane per pass: the fewest of 1, 2, 4, 8 that cover a token's
  // Hkv * D / 8 chunks in one pass (rows of more than 512 chunks take several).
  const int64_t per_tok = num_kv_heads * p.cpr;
  KernelTimer timer;
  const dim3 g((unsigned)grid), blk(kAThreads);
  if (per_tok <= 64)
    timer.launch(paged_append_kernel<1>, g, blk, 0, (hipStream_t)stream, p);
  else if (per_tok <= 128)
    timer.launch(paged_append_kernel<2>, g, blk, 0, (hipStream_t)stream, p);
  else if (per_tok <= 256)
    timer.launch(paged_append_kernel<4>, g, blk, 0, (hipStream_t)stream, p);
  else
    timer.launch(paged_append_kernel<8>, g, blk, 0, (hipStream_t)stream, p);
  return check_launch("paged_append_kernel");
}
