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
// Work: one thread per 16-byte chunk of one (token, kv head) row; a chunk of
// K and the matching chunk of V are moved together.  HBM-bound: 4 * D bytes
// per (token, kv head) (read K and V, write K and V).
#include "akt_common.hpp"
#include "akt_host.hpp"

namespace akt {
namespace {

constexpr int kAThreads = 256;

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

__global__ __launch_bounds__(kAThreads) void paged_append_kernel(AppendParams p) {
  const int64_t gt = (int64_t)blockIdx.x * kAThreads + threadIdx.x;
  const int64_t per_tok = (int64_t)p.Hkv * p.cpr;
  const int64_t tok = gt / per_tok;
  if (tok >= p.total_new) return;
  const int rem = (int)(gt - tok * per_tok);
  const int h = rem / p.cpr;
  const int c = rem - h * p.cpr;
  // Sequence of new row `tok`: last b with append_indptr[b] <= tok.
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.append_indptr[mid] <= tok) lo = mid;
    else hi = mid - 1;
  }
  const int b = lo;
  const int64_t a0 = p.append_indptr[b], a1 = p.append_indptr[b + 1];
  if (tok < a0 || tok >= a1) return;  // malformed indptr: nothing to write
  const int np = p.indptr[b + 1] - p.indptr[b];
  if (np <= 0) return;
  const int last = min(max(p.last_len[b], 0), p.page_size);
  const int64_t len = (int64_t)(np - 1) * p.page_size + last;
  const int64_t pos = len - (a1 - a0) + (tok - a0);
  if (pos < 0 || pos >= len) return;
  const int lp = (int)(pos / p.page_size);
  const int slot = (int)(pos - (int64_t)lp * p.page_size);
  const int page = p.indices[p.indptr[b] + lp];
  if (page < 0 || page >= p.num_pool_pages) return;
  const half_t* ks = p.k_new + tok * p.kn_st + (int64_t)h * p.kn_sh + 8 * c;
  const half_t* vs = p.v_new + tok * p.vn_st + (int64_t)h * p.vn_sh + 8 * c;
  half_t* dst = p.pool + (int64_t)page * p.sp + (int64_t)h * p.sh + (int64_t)slot * p.ss + 8 * c;
  const uint4_t kv = ld16(ks), vv = ld16(vs);
  st16(dst, kv);
  st16(dst + p.skv, vv);
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
  const int64_t threads = total_new * num_kv_heads * p.cpr;
  const int64_t grid = ceil_div(threads, kAThreads);
  AKT_CHECK(grid < (1ll << 31), "too many tokens");
  KernelTimer timer;
  timer.launch(paged_append_kernel, dim3((unsigned)grid), dim3(kAThreads), 0,
               (hipStream_t)stream, p);
  return check_launch("paged_append_kernel");
}
