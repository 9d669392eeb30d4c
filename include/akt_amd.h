/*
 * akt_amd.h - C ABI of the gfx950 attention kernel library (libakt_amd.so).
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * launches asynchronously on the given HIP stream (passed as void*; NULL is
 * the default stream) and returns AKT_OK or an error code; on error
 * akt_last_error() returns a message for the calling thread.  Nothing here
 * synchronises the stream or allocates device memory: the split-KV decode
 * entry points take a caller-owned workspace of the size reported by the
 * matching *_workspace_size() function.
 *
 * Workspace contract (all decode entry points): the first
 * min(AKT_WORKSPACE_ZERO_BYTES, workspace size) bytes hold scheduling and
 * per-unit arrival counters and must be zero before a workspace is first
 * used; every call leaves them zero again when it completes.  (The counters
 * of calls with more than 32768 units past that prefix are zero-filled by the
 * call itself.)  A workspace may be reused by any decode entry point, but
 * only by calls ordered on one stream (calls that overlap in time must use
 * different workspaces).
 *
 * Tensor element types: q/k/v/o and KV pools are IEEE fp16 (akt_prefill_fwd_ex
 * also takes bf16); page tables, kept-token indices and counts are int32;
 * MagicPIG K/L and LSE are fp32.
 * Strides are in elements.  The innermost (head_dim) stride must be 1 and
 * every row must start 16-byte aligned.
 *
 * Reference interfaces replaced (KiritoHugh/attention_kernel_triton):
 *   prefill_flash_attention.py:342                       flash_attention_prefill
 *   prefill_flash_attention_var_len_padding.py:348       flash_attention_prefill(varlen=)
 *   decode_flash_attention_redundant.py:233              flash_attention_decode
 *   decode_flash_attention_redundant_var_len_paged.py:228  flash_attention_decode_paged
 *   sparsetoken_decode_flash_attention_redundant.py:127  sparsetoken_flash_attention_decode
 *   sparsetoken_decode_flash_attention_redundant_var_len_paged.py:170
 *                                                        sparsetoken_flash_attention_decode_paged
 *   magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm.py:166
 *                                                        magicpig_sparsetoken_flash_attention_decode_paged
 *   sparsetoken_decode_flash_attention_redundant.py:283-295 (kept-index selection, harness code)
 *   prefill_flash_attention.py:331-334 (stubbed LSE store)  akt_prefill_fwd_lse, akt_merge_states
 *   sparse_decode_flash_attention.py:13-15 (CSR index note)   akt_sparse_decode_*csr_fwd
 *   decode_flash_attention_redundant_var_len_paged.py:349-353 (page tables, harness)
 *                                                        akt_paged_kv_append
 */
#ifndef AKT_AMD_H
#define AKT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKT_OK 0
#define AKT_ERR_INVALID_ARGUMENT 1 /* shape, stride, alignment or value check failed */
#define AKT_ERR_UNSUPPORTED 2      /* a valid request this build has no kernel for   */
#define AKT_ERR_WORKSPACE 3        /* workspace missing or smaller than required      */
#define AKT_ERR_HIP 4              /* the HIP runtime reported an error at launch     */

/* Element types for entry points that accept more than one. */
#define AKT_DTYPE_F16 0
#define AKT_DTYPE_F32 1
#define AKT_DTYPE_BF16 2

/* Message describing the last failure on the calling thread ("" if none). */
const char* akt_last_error(void);

/* ABI version of this header (bumped on any signature or contract change). */
#define AKT_ABI_VERSION 2
int akt_abi_version(void);

/* Bytes at the start of a decode workspace that must be zero before its first
 * use: a 256-byte counter header and 32768 int32 arrival counters. */
#define AKT_WORKSPACE_ZERO_BYTES (256u + 32768u * 4u)

/*
 * Causal / non-causal GQA prefill, O = softmax(scale * Q K^T [+ causal]) V.
 * Replaces prefill_flash_attention.py:342 and, with varlen != NULL,
 * prefill_flash_attention_var_len_padding.py:348.
 *   q, o: [batch, num_q_heads, seq_len, head_dim]; k, v: [batch, num_kv_heads,
 *   seq_len, head_dim]; q head h reads kv head h / (num_q_heads / num_kv_heads).
 *   varlen: optional device array [batch] of valid lengths (int32 when
 *   varlen_bits == 32, int64 when 64, ignored when varlen == NULL).  Query
 *   blocks of 64 rows that start at or beyond a sequence's length are not
 *   written (as in the reference); rows < length never read keys >= length
 *   when causal.
 *   head_dim: 64, 128, 192 or 256.
 */
int akt_prefill_fwd(const void* q, const void* k, const void* v, void* o,
                    int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                    int64_t seq_len, int64_t head_dim,
                    const int64_t q_stride[4], const int64_t k_stride[4],
                    const int64_t v_stride[4], const int64_t o_stride[4],
                    float softmax_scale, int causal,
                    const void* varlen, int varlen_bits, void* stream);

/*
 * akt_prefill_fwd plus the natural-log softmax normaliser of every computed
 * row: lse[b, h, s] = ln sum_k exp(scale * q_s . k) over the keys row s
 * attends (fp32, strides lse_stride[0..2] over batch, head, row).  Rows that
 * akt_prefill_fwd leaves unwritten are left unwritten here too.  The
 * reference computes the same quantity and leaves its store commented out
 * (prefill_flash_attention.py:331-334); this is its public form, for
 * chunked prefill and akt_merge_states.
 */
int akt_prefill_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse,
                        int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                        int64_t seq_len, int64_t head_dim,
                        const int64_t q_stride[4], const int64_t k_stride[4],
                        const int64_t v_stride[4], const int64_t o_stride[4],
                        const int64_t lse_stride[3], float softmax_scale, int causal,
                        const void* varlen, int varlen_bits, void* stream);

/*
 * akt_prefill_fwd / akt_prefill_fwd_lse for either element type: q, k, v and
 * o are all fp16 (dtype AKT_DTYPE_F16) or all bf16 (AKT_DTYPE_BF16); lse may
 * be NULL (no normaliser; lse_stride is then ignored).  With bf16 both MFMA
 * products run in bf16 and the probabilities are rounded to bf16 for P.V (the
 * fp16 path rounds them to fp16, as the reference's prefill does at
 * prefill_flash_attention.py:94).  The reference's prefill kernels take fp16
 * only (their P.V casts P to fp16); this entry point has no counterpart there.
 */
int akt_prefill_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse,
                       int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                       int64_t seq_len, int64_t head_dim,
                       const int64_t q_stride[4], const int64_t k_stride[4],
                       const int64_t v_stride[4], const int64_t o_stride[4],
                       const int64_t lse_stride[3], float softmax_scale, int causal,
                       const void* varlen, int varlen_bits, int dtype, void* stream);

/*
 * Merge attention states computed over disjoint key sets.  For each of
 * `rows` (query, head) rows and n_parts parts i:
 *   lse_out = ln sum_i exp(lse_i),  o_out = sum_i exp(lse_i - lse_out) o_i.
 * Parts with lse_i = -inf contribute nothing; a row with no contributing
 * part gets o_out = 0 and lse_out = -inf.  No reference counterpart: it is
 * the combine the reference's stubbed LSE stores
 * (prefill_flash_attention.py:331-334, decode_flash_attention_redundant.py:225-228)
 * would feed, for chunked prefill / decode and per-GPU shards.
 *   o_parts: [n_parts, rows, head_dim] of type o_parts_dtype (AKT_DTYPE_F16 or
 *   AKT_DTYPE_F32), strides o_parts_stride[0..1] (head_dim stride 1);
 *   lse_parts: fp32 [n_parts, rows], strides lse_parts_stride[0..1];
 *   o_out: [rows, head_dim] of type o_out_dtype, row stride o_out_row_stride;
 *   lse_out: optional fp32 [rows], stride lse_out_row_stride.
 *   head_dim: a multiple of 8 up to 512.
 */
int akt_merge_states(const void* o_parts, int o_parts_dtype, const float* lse_parts,
                     void* o_out, int o_out_dtype, float* lse_out, int64_t n_parts,
                     int64_t rows, int64_t head_dim, const int64_t o_parts_stride[2],
                     const int64_t lse_parts_stride[2], int64_t o_out_row_stride,
                     int64_t lse_out_row_stride, void* stream);

/*
 * Single-token GQA decode over a dense cache.  Replaces
 * decode_flash_attention_redundant.py:233.
 *   q: [batch, num_q_heads, 1, head_dim] (strides q_stride[0], [1], -, [3]);
 *   k, v: [batch, num_kv_heads, seq_len, head_dim];
 *   o: contiguous [batch, num_q_heads, head_dim] fp16;
 *   lse: optional contiguous [batch, num_q_heads] fp32 (natural log of the
 *   softmax normaliser of the scaled scores).  head_dim: 64, 128 or 256.
 *   chunk_tokens: split-KV chunk length: 128, 256, 512 or 640 tokens, 0 = automatic
 *   (a hint: pages that do not hold whole 16-token groups, and paged batches
 *   over 1024 sequences, use 256).
 */
size_t akt_decode_workspace_size(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                 int64_t seq_len, int64_t head_dim, int64_t chunk_tokens);
int akt_decode_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                   int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                   int64_t seq_len, int64_t head_dim,
                   const int64_t q_stride[4], const int64_t k_stride[4],
                   const int64_t v_stride[4], float softmax_scale, int64_t chunk_tokens,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Paged var-len GQA decode.  Replaces
 * decode_flash_attention_redundant_var_len_paged.py:228.
 *   kv_cache: [num_pool_pages, 2, num_kv_heads, page_size, head_dim] (K at
 *   [:,0], V at [:,1]) with strides kv_stride[5];
 *   kv_page_indptr [batch+1], kv_page_indices [total_pages],
 *   kv_last_page_len [batch]: int32 CSR page table.  Sequence b has
 *   (indptr[b+1]-indptr[b]-1)*page_size + last_page_len[b] tokens (0 when it
 *   has no pages; last_page_len is clamped to [0, page_size]).  Page ids
 *   outside [0, num_pool_pages) are skipped.
 *   o: contiguous [batch, num_q_heads, head_dim]; lse optional [batch, num_q_heads].
 *   chunk_tokens 0 (automatic) runs the stream-K kernel when batch <= 1024
 *   and page_size is a multiple of 16: every wave of the launch takes a fixed
 *   range of 16-token groups, and its workspace holds one partial per wave
 *   the device keeps resident plus one per (sequence, head group), so the
 *   workspace size depends on the current device.  Otherwise, and for the
 *   explicit lengths 128, 256, 512 or 640, the chunked split kernel runs.
 */
size_t akt_decode_paged_workspace_size(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                       int64_t head_dim, int64_t page_size, int64_t total_pages,
                                       int64_t chunk_tokens);
int akt_decode_paged_fwd(const void* q, const void* kv_cache, const int32_t* kv_page_indptr,
                         const int32_t* kv_page_indices, const int32_t* kv_last_page_len,
                         void* o, float* lse, int64_t batch, int64_t num_q_heads,
                         int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                         int64_t total_pages, int64_t num_pool_pages,
                         const int64_t q_stride[4], const int64_t kv_stride[5],
                         float softmax_scale, int64_t chunk_tokens,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * akt_decode_paged_fwd without a workspace argument: no reference
 * counterpart.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc), and it allocates nothing.  The split-KV workspace is a
 * file-scope device array of AKT_NOALLOC_SCRATCH_BYTES that every GPU the
 * library runs on holds until the process ends; its counter area is
 * zero-filled (by a fill kernel on `stream`) at the first call on a device,
 * and every launch leaves its counters at zero again.  A call whose workspace
 * (akt_decode_paged_workspace_size of the same arguments) exceeds the array
 * fails with AKT_ERR_INVALID_ARGUMENT.  All calls on one GPU share the array:
 * calls that overlap in time on one GPU race, so order them (one stream).
 * Results are bit-identical to akt_decode_paged_fwd's.
 */
#define AKT_NOALLOC_SCRATCH_BYTES (32u << 20)
int akt_decode_paged_fwd_noalloc(const void* q, const void* kv_cache,
                                 const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                 const int32_t* kv_last_page_len, void* o, float* lse,
                                 int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                 int64_t head_dim, int64_t page_size, int64_t total_pages,
                                 int64_t num_pool_pages, const int64_t q_stride[4],
                                 const int64_t kv_stride[5], float softmax_scale,
                                 int64_t chunk_tokens, void* stream);

/*
 * Sparse-token decode over a dense cache.  Replaces
 * sparsetoken_decode_flash_attention_redundant.py:127.
 *   sparse_ind: [batch, num_q_heads, l_max] int32 kept token indices
 *   (ascending in the reference harness; order does not matter here), entry
 *   i is used when i < sparse_nnz[b, h] (nnz is clamped to [0, l_max]).
 *   Indices outside [0, seq_len) are skipped.  A head with no kept tokens
 *   produces o = 0 and lse = -inf.
 *   ind_stride: strides of sparse_ind over (batch, head) (last stride 1);
 *   nnz_stride: strides of sparse_nnz over (batch, head).
 */
size_t akt_sparse_decode_workspace_size(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                        int64_t l_max, int64_t num_splits);
int akt_sparse_decode_fwd(const void* q, const void* k, const void* v,
                          const int32_t* sparse_ind, const int32_t* sparse_nnz,
                          void* o, float* lse, int64_t batch, int64_t num_q_heads,
                          int64_t num_kv_heads, int64_t seq_len, int64_t head_dim, int64_t l_max,
                          const int64_t q_stride[4], const int64_t k_stride[4],
                          const int64_t v_stride[4], const int64_t ind_stride[2],
                          const int64_t nnz_stride[2], float softmax_scale, int64_t num_splits,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sparse-token decode over a paged var-len cache.  Replaces
 * sparsetoken_decode_flash_attention_redundant_var_len_paged.py:170.
 * Kept token t of sequence b lives in page
 * kv_page_indices[kv_page_indptr[b] + t / page_size], slot t % page_size.
 * Tokens whose logical page is outside the sequence's page list, or whose
 * page id is outside [0, num_pool_pages), are skipped.
 */
int akt_sparse_decode_paged_fwd(const void* q, const void* kv_cache,
                                const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                const int32_t* sparse_ind, const int32_t* sparse_nnz,
                                void* o, float* lse, int64_t batch, int64_t num_q_heads,
                                int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_pool_pages, int64_t l_max,
                                const int64_t q_stride[4], const int64_t kv_stride[5],
                                const int64_t ind_stride[2], const int64_t nnz_stride[2],
                                float softmax_scale, int64_t num_splits,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * MagicPIG "with norm" sparse paged decode.  Replaces
 * magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm.py:166.
 * Score of kept token i: q.k_i / sqrt(head_dim) - ln(u_i) with
 *   c = q.k_i / (|q| |k_i| + 1e-8) clamped to [-1+1e-7, 1-1e-7],
 *   p = clamp(1 - acos(c)/pi, 0, 1), x = p^K,
 *   u = max(1 - (1-x)^L - L x (1-x)^(L-1), 1e-10),
 * with per-(batch, q head) K, L: contiguous fp32 [batch, num_q_heads].  u is
 * evaluated in fp32 in the equal form -expm1((L-1) g(-x) + g((L-1) x)),
 * g(y) = log1p(y) - y, which does not cancel for x in [0, 1) and L >= 1 (a
 * few fp32 ulps of relative error in u); x >= 1 or (L-1) x <= -1 fall back to
 * the formula as written.
 * Workspace size: akt_sparse_decode_workspace_size().
 */
int akt_magicpig_decode_paged_fwd(const void* q, const void* kv_cache,
                                  const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                  const int32_t* sparse_ind, const int32_t* sparse_nnz,
                                  const float* lsh_k, const float* lsh_l,
                                  void* o, float* lse, int64_t batch, int64_t num_q_heads,
                                  int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                  int64_t num_pool_pages, int64_t l_max,
                                  const int64_t q_stride[4], const int64_t kv_stride[5],
                                  const int64_t ind_stride[2], const int64_t nnz_stride[2],
                                  int64_t num_splits, void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * Sparse-token decode with kept indices in CSR form (inds + ptr) instead of
 * the -1-padded [batch, num_q_heads, l_max] rows: row u = b * num_q_heads + h
 * keeps the tokens inds[ptr[u] .. ptr[u+1]) (int32 token positions, int64
 * row pointer [batch * num_q_heads + 1]).  The second index format proposed
 * in sparse_decode_flash_attention.py:13-15 (no padding, no l_max); results
 * equal akt_sparse_decode_fwd on the same kept tokens.  max_nnz is a planning
 * hint (the longest row) for the automatic split count and the workspace size
 * (akt_sparse_decode_workspace_size with l_max = max_nnz); rows of any length
 * are handled.  Other arguments as akt_sparse_decode_fwd.
 */
int akt_sparse_decode_csr_fwd(const void* q, const void* k, const void* v, const int32_t* inds,
                              const int64_t* ptr, void* o, float* lse, int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                              int64_t head_dim, int64_t max_nnz, const int64_t q_stride[4],
                              const int64_t k_stride[4], const int64_t v_stride[4],
                              float softmax_scale, int64_t num_splits, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Sparse paged decode (and, with lsh_k / lsh_l given, the MagicPIG with-norm
 * variant) with CSR kept indices; see akt_sparse_decode_csr_fwd for the CSR
 * format and akt_sparse_decode_paged_fwd / akt_magicpig_decode_paged_fwd for
 * the rest.  Scale 1/sqrt(head_dim).
 */
int akt_sparse_decode_paged_csr_fwd(const void* q, const void* kv_cache,
                                    const int32_t* kv_page_indptr, const int32_t* kv_page_indices,
                                    const int32_t* inds, const int64_t* ptr, const float* lsh_k,
                                    const float* lsh_l, void* o, float* lse, int64_t batch,
                                    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                    int64_t page_size, int64_t num_pool_pages, int64_t max_nnz,
                                    const int64_t q_stride[4], const int64_t kv_stride[5],
                                    int64_t num_splits, void* workspace, size_t workspace_bytes,
                                    void* stream);

/*
 * Paged KV cache write side: append new tokens into the page pool.
 * Sequence b's n_b = append_indptr[b+1] - append_indptr[b] new tokens
 * (rows of k_new / v_new: [total_new, num_kv_heads, head_dim], strides
 * *_new_stride[0..2]) become the last n_b logical positions of b under the
 * page table kv_page_indptr / kv_page_indices / kv_last_page_len, which must
 * already include them (see attention_kernel_triton_amd.paged_kv.PagedKVCache).
 * Writes pool[page, 0, h, slot] (K) and pool[page, 1, h, slot] (V) with the
 * decode kernels' addressing; tokens whose position or page id is outside
 * the table or pool are skipped.  No reference counterpart: the reference's
 * tests build page tables by hand
 * (decode_flash_attention_redundant_var_len_paged.py:349-353).
 */
int akt_paged_kv_append(const void* k_new, const void* v_new, const int32_t* append_indptr,
                        void* kv_cache, const int32_t* kv_page_indptr,
                        const int32_t* kv_page_indices, const int32_t* kv_last_page_len,
                        int64_t batch, int64_t total_new, int64_t num_kv_heads,
                        int64_t head_dim, int64_t page_size, int64_t num_pool_pages,
                        const int64_t k_new_stride[3], const int64_t v_new_stride[3],
                        const int64_t kv_stride[5], void* stream);

/*
 * Kept-token index selection (the reference harness step at
 * sparsetoken_decode_flash_attention_redundant.py:283-295 and
 * sparsetoken_decode_flash_attention_redundant_var_len_paged.py:341-353).
 * For each of `rows` rows: kept = {j < n_r : keep(r, j)} in ascending order,
 * where n_r = row_len[r] (or n when row_len == NULL) and keep(r, j) is
 *   mask[r * mask_row_stride + j] != 0            (akt_kept_index_from_mask)
 *   uniform[r * row_stride + j] < kept_ratio      (akt_kept_index_from_uniform)
 * If ensure_nonempty and nothing is kept, index 0 is kept.
 * Writes sparse_ind[r * l_max + i] = kept[i] for i < min(|kept|, l_max) and -1
 * for the rest of the row, and sparse_nnz[r] = |kept|.
 */
int akt_kept_index_from_mask(const uint8_t* mask, int64_t rows, int64_t n,
                             int64_t mask_row_stride, const int32_t* row_len,
                             int32_t* sparse_ind, int64_t l_max, int32_t* sparse_nnz,
                             int ensure_nonempty, void* stream);
int akt_kept_index_from_uniform(const float* uniform, float kept_ratio, int64_t rows, int64_t n,
                                int64_t row_stride, const int32_t* row_len,
                                int32_t* sparse_ind, int64_t l_max, int32_t* sparse_nnz,
                                int ensure_nonempty, void* stream);

/*
 * Kernel timer (diagnostics; no counterpart in the reference, which times
 * whole Python calls with triton.testing.do_bench).  While enabled, every
 * entry point above records a HIP event pair around its dominant kernel on
 * the launch stream.  akt_kernel_timer_read() waits for the recorded events
 * and returns the summed elapsed milliseconds and the number of launches;
 * akt_kernel_timer_enable() discards what was recorded.
 */
int akt_kernel_timer_enable(int enable);
int akt_kernel_timer_read(double* total_ms, int64_t* launches);

/*
 * Read-rate ceilings (diagnostics; no counterpart in the reference, which has
 * no bandwidth model).  They measure, on the caller's data, how fast the
 * device streams the bytes a paged decode reads, with no arithmetic:
 *   akt_diag_paged_gather reads the K and V block (page_size x head_dim fp16,
 *   contiguous: kv_stride[3] == head_dim) of every (CSR page position, kv
 *   head) pair of kv_page_indices[0 .. total_pages), as the decode kernels
 *   address them (page ids outside [0, num_pool_pages) read page 0); blocks
 *   of 2, 4, 8 or 16 KB.
 *   akt_diag_stream_read reads `bytes` (a multiple of 16) from `data` in order.
 * Both write nothing but possibly one word of `sink` (a device uint32).
 */
int akt_diag_paged_gather(const void* kv_cache, const int32_t* kv_page_indices,
                          int64_t total_pages, int64_t num_kv_heads, int64_t head_dim,
                          int64_t page_size, int64_t num_pool_pages, const int64_t kv_stride[5],
                          uint32_t* sink, void* stream);
int akt_diag_stream_read(const void* data, int64_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AKT_AMD_H */
