/*
 * kessie_mi355x.h -- C ABI of libkessie_mi355x.so, the MI355X (gfx950) build of
 * KeSSie's long-context attention hot path: fog attention (paged decode and
 * chunked prefill), RoPE position remap of recalled K, and paged-KV
 * insert / evict / compact / gather.
 *
 * Conventions (all entry points):
 *   - Every pointer argument is a DEVICE pointer unless stated otherwise; the
 *     caller owns all memory.  Nothing here allocates device memory.
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).  Calls
 *     are asynchronous on that stream; none of them synchronises the device.
 *   - The `kessie_*` entry points return an int status (KESSIE_OK == 0) and
 *     never print.  On failure, kessie_get_last_error() returns the message
 *     (thread-local).  Argument errors are detected on the host before any
 *     launch, so a failed call has launched nothing.
 *   - The five `launch_kessie_*` entry points keep the reference's exact
 *     signatures and `void` return; they record errors through the same
 *     thread-local message instead of printing to stderr.
 *   - Page layout ("native"): pool[num_pages][page_size][2 (K,V)][Hkv][D];
 *     other layouts (e.g. vLLM's [2][blocks][P][Hkv][D]) are described by the
 *     element strides page_stride / tok_stride / kv_stride / head_stride, with
 *     the innermost (D) dimension contiguous.
 */
#ifndef KESSIE_MI355X_H
#define KESSIE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; these entry points are its
 * only exports. */
#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

/* Element type codes. */
#define KESSIE_DTYPE_F32 0
#define KESSIE_DTYPE_BF16 1
#define KESSIE_DTYPE_F16 2

/* Status codes. */
#define KESSIE_OK 0
#define KESSIE_ERR_INVALID 1     /* bad argument (null pointer, size, stride) */
#define KESSIE_ERR_UNSUPPORTED 2 /* valid but not implemented (dtype, shape)  */
#define KESSIE_ERR_WORKSPACE 3   /* workspace missing or too small            */
#define KESSIE_ERR_HIP 4         /* the HIP runtime reported an error         */

/* Copies the calling thread's last error message (NUL-terminated, truncated
 * to `cap` bytes) into host buffer `buf`; returns the last status code. */
int kessie_get_last_error(char* buf, size_t cap);

/* Library version as major*10000 + minor*100 + patch. */
int kessie_version(void);

/* =========================================================================
 * Legacy entry points -- identical signatures to the reference launchers.
 *
 * The two dense launchers take no workspace, so when a key split pays (small
 * grids with causal imbalance) they keep one partial buffer per (device,
 * stream), allocated on the first such call on that stream outside graph
 * capture, grown on a larger request (the old buffer kept), never freed
 * before process exit.  A call that would need a new buffer while its
 * stream is capturing, or more than 1 GiB of partials, runs unsplit.
 * ========================================================================= */

/* Dense windowed attention, fp16 [B,H,N,D] Q/K/V/O, D in {64,128}.
 * Semantics of the reference's torch math (kessie_hip_kernels.py:577-589):
 * causal mask j<=i, window keeps 0<=i-j<W (W=0: full).
 * Replaces kessie_kernels_v2.hip:716-751 (launch_kessie_windowed_attn). */
void launch_kessie_windowed_attn(const void* Q, const void* K, const void* V,
                                 void* O, float sm_scale, int batch_size,
                                 int num_heads, int seq_len, int head_dim,
                                 int window_size, int is_causal, void* stream);

/* Dense attention with fog weights scaling V rows: O = softmax(QK^T s) (w.V),
 * fog_weights fp32 [N] (kessie_hip_kernels.py:592-593).
 * Replaces kessie_kernels_v2.hip:788-825 (launch_kessie_fused_fog_attn). */
void launch_kessie_fused_fog_attn(const void* Q, const void* K, const void* V,
                                  void* O, const void* fog_weights,
                                  float sm_scale, int batch_size, int num_heads,
                                  int seq_len, int head_dim, int window_size,
                                  int is_causal, void* stream);

/* Threshold eviction: valid[p]==1 && positions[p] < thr  ->  valid[p]=0 and
 * *evict_count += 1 (caller zeroes the counter).  int8 valid, int32 positions.
 * Replaces kessie_kernels_v2.hip:753-764 (launch_kessie_page_evict). */
void launch_kessie_page_evict(void* page_valid, const void* page_positions,
                              void* evict_count, int evict_before_pos,
                              int num_pages, void* stream);

/* Scatter new fp16 K/V [T,H,D] into the native fp16 pool at target pages
 * (token t -> page target_page_ids[t/P], slot t%P); sets valid=1 and
 * positions = conv_pos + t for each page's slot-0 token; page ids outside
 * [0,max_pages) are skipped.
 * Replaces kessie_kernels_v2.hip:766-782 (launch_kessie_page_insert). */
void launch_kessie_page_insert(void* kv_cache, const void* new_keys,
                               const void* new_values,
                               const void* target_page_ids, void* page_valid,
                               void* page_positions, int conv_pos,
                               int num_tokens, int num_heads, int head_dim,
                               int page_size, int max_pages, void* stream);

/* In-place RoPE remap of fp16 K [T,H,2*half_dim] from orig to target
 * positions (rotate-half pairs (d, d+half)).
 * Replaces kessie_kernels_v2.hip:827-842 (launch_kessie_rope_remap). */
void launch_kessie_rope_remap(void* k_data, const void* orig_positions,
                              const void* target_positions, float rope_theta,
                              int num_tokens, int num_heads, int half_dim,
                              void* stream);

/* =========================================================================
 * Paged fog attention
 * ========================================================================= */

/* Bytes of workspace kessie_fog_decode_paged needs for these sizes (host
 * call, no device work).  max_ctx is the largest ctx_lens[b]. */
size_t kessie_fog_decode_workspace_bytes(int batch, int num_q_heads,
                                         int num_kv_heads, int head_dim,
                                         int max_ctx, int page_size, int dtype);

/* Decode (one query token per sequence) over paged KV, GQA
 * (q head h uses kv head h / (Hq/Hkv)).  Sequence b holds ctx_lens[b] tokens
 * at positions 0..ctx-1; token t lives in page page_table[b*table_stride +
 * t/page_size], slot t%page_size.  The query sits at position ctx-1.
 *   scores  s_j = (q . k_j) * sm_scale [+ fog_bias[b*fog_bias_bstride + j]]
 *   mask    j < ctx and (window == 0 or (ctx-1) - j < window)
 *   output  o = sum_j softmax(s)_j * w_j * v_j,  w_j = fog_vscale[b*bstride+j]
 *           (w == 1 when fog_vscale is NULL; the sum is not renormalised).
 * q/out: [B][Hq][D] contiguous in `dtype`; pool elements in `dtype`;
 * accumulation in fp32.  Page ids outside [0,num_pages) mask their tokens.
 * A sequence with no visible key yields a zero output row.  The fog semantics follow kessie_hip_kernels.py:
 * 577-593 (V mode) and kessie_attention.py:114-139 (bias mode).  The
 * reference has no paged/GQA decode kernel; the GPU launcher it stands in
 * for is kessie_kernels_v2.hip:788-825. */
int kessie_fog_decode_paged(
    const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
    int64_t tok_stride,
    int64_t kv_stride, int64_t head_stride, const int32_t* page_table,
    int64_t table_stride, const int32_t* ctx_lens, const float* fog_vscale,
    int64_t fog_vscale_bstride, const float* fog_bias, int64_t fog_bias_bstride,
    void* out, int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int page_size, int max_ctx, int window, float sm_scale, int dtype,
    void* workspace, size_t workspace_bytes, void* stream);

/* Size of the static device scratch of kessie_fog_decode_paged_noalloc. */
#define KESSIE_DECODE_NOALLOC_SCRATCH_BYTES (16u << 20)

/* kessie_fog_decode_paged without a workspace argument, allocating nothing:
 * the split partials go to a static device array of
 * KESSIE_DECODE_NOALLOC_SCRATCH_BYTES (16 MiB) per GPU, held until the
 * process ends.  Same arguments (minus workspace / workspace_bytes),
 * semantics and results, bit for bit, as kessie_fog_decode_paged.  Returns
 * KESSIE_ERR_WORKSPACE, launching nothing, when the partials of these sizes
 * exceed the array (B * Hq * S * (head_dim + 2) * 4 bytes plus alignment, S =
 * kessie_fog_decode_num_splits(...)).  Calls that overlap on one GPU share
 * the array and race: serialise them (one stream, or events).  The first
 * call on a device looks the array's address up (hipGetSymbolAddress); make
 * it outside HIP graph capture, after which the call may be captured and
 * replayed.  No
 * counterpart in the reference: it exists for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid allocation). */
int kessie_fog_decode_paged_noalloc(
    const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
    int64_t tok_stride, int64_t kv_stride, int64_t head_stride,
    const int32_t* page_table, int64_t table_stride, const int32_t* ctx_lens,
    const float* fog_vscale, int64_t fog_vscale_bstride, const float* fog_bias,
    int64_t fog_bias_bstride, void* out, int batch, int num_q_heads,
    int num_kv_heads, int head_dim, int page_size, int max_ctx, int window,
    float sm_scale, int dtype, void* stream);

/* Number of key splits S the decode uses for these sizes (host call). */
int kessie_fog_decode_num_splits(int batch, int num_kv_heads, int max_ctx,
                                 int page_size);

/* First half of kessie_fog_decode_paged: the streaming kernel only.  Writes
 * the per-split partials of every row r = b*Hq + h into the workspace:
 *   o[r][s][D] fp32 (unnormalised sum of p*w*v), then, each starting on a
 *   256-byte boundary, m[r][s] (running max, -inf when the split saw no key)
 *   and l[r][s] (sum of p), with S = kessie_fog_decode_num_splits(...).
 * Always writes partials, also when S == 1.  These are also the (m, l, o)
 * triples a context-parallel split of one sequence across devices would
 * exchange before kessie_fog_decode_combine.  (No reference counterpart: the
 * reference has no split decode.) */
int kessie_fog_decode_partials(
    const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
    int64_t tok_stride, int64_t kv_stride, int64_t head_stride,
    const int32_t* page_table, int64_t table_stride, const int32_t* ctx_lens,
    const float* fog_vscale, int64_t fog_vscale_bstride, const float* fog_bias,
    int64_t fog_bias_bstride, int batch, int num_q_heads, int num_kv_heads,
    int head_dim, int page_size, int max_ctx, int window, float sm_scale,
    int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Second half: merges the partials in `workspace` (laid out as above) into
 * out [B][Hq][D] in `dtype`: o = sum_s e_s o_s / sum_s e_s l_s with
 * e_s = exp(m_s - max_s m_s); rows with no key get zeros. */
int kessie_fog_decode_combine(const void* workspace, size_t workspace_bytes,
                              void* out, int batch, int num_q_heads,
                              int num_kv_heads, int head_dim, int max_ctx,
                              int page_size, int dtype, void* stream);

/* Bytes of workspace kessie_fog_prefill_paged may need (host call): room for
 * per-split partials at the largest of the kernels' split counts.  The MFMA
 * kernels (bf16/fp16, and fp32 with head_dim 128) touch it only when a small
 * chunk on a long context splits the key range (S from the CU count, or
 * KESSIE_PREFILL_SPLITS); the generic kernel always uses it. */
size_t kessie_fog_prefill_workspace_bytes(int batch, int num_q_tokens,
                                          int num_q_heads, int num_kv_heads,
                                          int head_dim, int max_ctx,
                                          int page_size, int dtype);

/* Chunked prefill: C query tokens per sequence appended after L prior tokens
 * (ctx_lens[b] = L + C counts them all; the chunk's K/V are already in the
 * pool).  Query i (0<=i<C) sits at position q_pos = ctx-C+i and attends keys
 * j <= q_pos (causal) with (window == 0 or q_pos - j < window), fog as in
 * decode, fog index = key position.  q/out: [B][C][Hq][D] contiguous.  This
 * equals the last C rows of the reference's dense math over ctx tokens
 * (kessie_hip_kernels.py:577-593).  Kernels: bf16/fp16 on MFMA (head_dim 128,
 * pages of 16 * 2^k tokens, GQA 1/2/4/8/16), fp32 on fp32 MFMA (head_dim 128,
 * same pages, GQA up to 128), everything else on the generic kernel. */
int kessie_fog_prefill_paged(
    const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
    int64_t tok_stride,
    int64_t kv_stride, int64_t head_stride, const int32_t* page_table,
    int64_t table_stride, const int32_t* ctx_lens, const float* fog_vscale,
    int64_t fog_vscale_bstride, const float* fog_bias, int64_t fog_bias_bstride,
    void* out, int batch, int num_q_tokens, int num_q_heads, int num_kv_heads,
    int head_dim, int page_size, int max_ctx, int window, float sm_scale,
    int causal, int dtype, void* workspace, size_t workspace_bytes,
    void* stream);

/* The same chunked prefill for a batch whose sequences have different chunk
 * lengths, in one launch (the prefill half of a mixed serving batch, which
 * KeSSieAttentionImpl.forward, kessie_attention.py:278-304, hands to one
 * attention call): sequence b's queries are rows query_start_loc[b] -
 * query_start_loc[0] .. query_start_loc[b+1] - query_start_loc[0] - 1 of
 * q/out ([T][Hq][D] contiguous; query_start_loc int32 [batch+1],
 * non-decreasing, on the device, e.g. a slice of vLLM's), chunk length C_b = query_start_loc[b+1] -
 * query_start_loc[b] <= max_query_len, query i of it at ctx_lens[b] - C_b + i
 * (a longer chunk is read as its first max_query_len queries at positions
 * ctx_lens[b] - max_query_len + i; its other rows are not written).
 * MFMA shapes only (head_dim 128, pages of 16 * 2^k tokens, 16-byte aligned
 * rows; bf16/fp16 with GQA 1/2/4/8/16, or fp32 on the fp32 MFMA kernel with
 * any GQA ratio up to 128); other shapes return KESSIE_ERR_UNSUPPORTED without
 * launching (call kessie_fog_prefill_paged per sequence instead).  The
 * workspace is sized by kessie_fog_prefill_workspace_bytes(batch,
 * max_query_len, ...) and used only when the chunks are too few to fill the
 * device (split-K). */
int kessie_fog_prefill_varlen(
    const void* q, const int32_t* query_start_loc, int max_query_len,
    const void* kv_pool, int num_pages, int64_t page_stride, int64_t tok_stride,
    int64_t kv_stride, int64_t head_stride, const int32_t* page_table,
    int64_t table_stride, const int32_t* ctx_lens, const float* fog_vscale,
    int64_t fog_vscale_bstride, const float* fog_bias, int64_t fog_bias_bstride,
    void* out, int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int page_size, int max_ctx, int window, float sm_scale, int causal,
    int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* =========================================================================
 * RoPE position remap
 * ========================================================================= */

/* In-place remap of K from orig_pos[t] to tgt_pos[t] for T tokens.  Token t's
 * K row is at  kv_pool + page*page_stride + (t%page_size)*tok_stride  with
 * page = page_list[t/page_size]; page_list == NULL means dense rows
 * (row t at t*tok_stride).  Heads at head_stride, D contiguous, D even.
 * inv_freq: fp32 [D/2] device table (the caller builds it exactly as
 * 1/(theta ** (arange(D/2)/(D/2))), kessie_hip_kernels.py:600).
 * Angle = float(tgt-orig) * inv_freq[j] (one fp32 multiply); the rotation
 * of pair (j, j+D/2) is computed in fp32 without fused multiply-add and
 * rounded to `dtype` (kessie_hip_kernels.py:596-606).  Tokens whose page id
 * lies outside [0,num_pages) are left untouched. */
int kessie_rope_remap_paged(void* kv_pool, int64_t page_stride,
                            int64_t tok_stride, int64_t head_stride,
                            const int32_t* page_list, int num_pages,
                            const int32_t* orig_pos, const int32_t* tgt_pos,
                            const float* inv_freq, int num_tokens,
                            int num_heads, int head_dim, int page_size,
                            int dtype, void* stream);

/* =========================================================================
 * Paged-KV management
 * ========================================================================= */

/* Insert T recalled tokens' K/V ([T][H][D] each, contiguous, `dtype`) into
 * the pool at target_pages (token t -> page target_pages[t/P], slot t%P);
 * page ids outside [0,num_pages) are skipped; for every inserted page the
 * slot-0 token sets page_valid=1, page_positions=conv_pos+t
 * (kessie_kernels_v2.hip:414-456 addressing).  When orig_pos/tgt_pos/inv_freq
 * are all non-NULL, K is RoPE-remapped on the way in (same arithmetic as
 * kessie_rope_remap_paged); otherwise it is copied unchanged. */
int kessie_page_insert_paged(void* kv_pool, int64_t page_stride,
                             int64_t tok_stride, int64_t kv_stride,
                             int64_t head_stride, const void* new_k,
                             const void* new_v, const int32_t* target_pages,
                             int8_t* page_valid, int32_t* page_positions,
                             int conv_pos, const int32_t* orig_pos,
                             const int32_t* tgt_pos, const float* inv_freq,
                             int num_tokens, int num_heads, int head_dim,
                             int page_size, int num_pages, int dtype,
                             void* stream);

/* Threshold eviction that also reports WHICH pages were freed, in ascending
 * physical id order (the order KeSSiePagedKVCache.evict_before appends them to
 * its free list, kessie_hip_kernels.py:526-540).  A page is freed when
 * page_valid==1 && positions < thr, or, when `allocated` is non-NULL, when it
 * is allocated (allocated[p]!=0) but not valid; freed pages get
 * page_valid=0 and allocated=0.  Writes the ids to freed_list[0..n) and n to
 * *freed_count.  Workspace: kessie_page_workspace_bytes(num_pages). */
int kessie_page_evict_list(int8_t* page_valid, const int32_t* page_positions,
                           int8_t* allocated, int evict_before_pos,
                           int num_pages, int32_t* freed_list,
                           int32_t* freed_count, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Bytes of workspace the page-management calls need for num_pages (host). */
size_t kessie_page_workspace_bytes(int num_pages);

/* Prepares a page workspace (any size from kessie_page_workspace_bytes) for
 * kessie_page_select_evict / kessie_page_evict_compact: their scratch, at the
 * start of the workspace, must hold this state on entry, and each call leaves
 * it so again.  Call once per workspace allocation, on the stream that will
 * use it (one fill launch).  A select call on a workspace that was never
 * initialised writes -2 to its counts and touches nothing else.  (No
 * reference counterpart: the reference's eviction needs no workspace.) */
int kessie_page_workspace_init(void* workspace, size_t workspace_bytes,
                               void* stream);

/* Score eviction: among pages with page_valid==1, evict the k with the
 * smallest keys (score[p], p) under the total order score ascending, then
 * page id ascending (scores compared as IEEE floats, -0 == +0, NaN not
 * allowed).  k = k_evict when k_evict >= 0 (clamped to the valid count),
 * else floor(evict_fraction * n_valid) computed in double.  Evicted pages get
 * page_valid=0; their ids go to evict_list ascending; k to *evict_count.
 * Deterministic: no order depends on atomics.  One launch whose workgroups
 * meet at bounded grid barriers: if the device could not run them at once,
 * *evict_count reads -1 and nothing else is written (page_valid and
 * evict_list are left as they were, so the call can be retried); the
 * workspace must have been prepared by
 * kessie_page_workspace_init (-2 otherwise).  num_pages below 2^29 (else
 * KESSIE_ERR_UNSUPPORTED).  (The reference only has the threshold predicate,
 * kessie_kernels_v2.hip:393-407; this applies it with an exact
 * k-th-order-statistic threshold.) */
int kessie_page_select_evict(const float* scores, int8_t* page_valid,
                             int num_pages, int k_evict, float evict_fraction,
                             int32_t* evict_list, int32_t* evict_count,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* Compaction of S page tables [S][table_stride] with lens[s] used entries:
 * survivors (page_valid[id]==1) keep their logical order; new_tables[s][0..n)
 * holds them, entries [n, table_stride) are set to -1, new_lens[s]=n.
 * gather_idx receives all survivors in (sequence, logical) order and
 * *gather_count their number.  Entries outside [0,num_pages) count as not
 * surviving.  Workspace: kessie_page_workspace_bytes(S*table_stride). */
int kessie_page_compact(const int32_t* tables, const int32_t* lens,
                        const int8_t* page_valid, int32_t* new_tables,
                        int32_t* new_lens, int32_t* gather_idx,
                        int32_t* gather_count, int num_seqs, int table_stride,
                        int num_pages, void* workspace, size_t workspace_bytes,
                        void* stream);

/* kessie_page_select_evict followed by kessie_page_compact of the tables by
 * the post-eviction valid flags, in one launch instead of two calls' worth:
 * every output equals what those two calls produce (evict_list / evict_count /
 * page_valid as select_evict; new_tables / new_lens / gather_idx /
 * gather_count as compact).  num_seqs <= 8192, num_pages and table_stride
 * below 2^29 (else KESSIE_ERR_UNSUPPORTED).
 * Workspace: kessie_page_workspace_bytes(max(num_pages, num_seqs)), prepared
 * by kessie_page_workspace_init (else both counts read -2).  The launch's
 * workgroups (at most 64) wait for each other at bounded grid barriers; if
 * the device cannot run them at once the wait runs out (~0.1 s each),
 * *evict_count and *gather_count read -1 and no other output is written
 * (page_valid, evict_list, new_tables, new_lens and gather_idx are left as
 * they were, so the call can be retried).  (The reference evicts by threshold only and compacts nothing,
 * kessie_hip_kernels.py:526-564; the caller this serves is the page
 * manager's evict-then-gather step.) */
int kessie_page_evict_compact(const float* scores, int8_t* page_valid,
                              int num_pages, int k_evict, float evict_fraction,
                              int32_t* evict_list, int32_t* evict_count,
                              const int32_t* tables, const int32_t* lens,
                              int num_seqs, int table_stride,
                              int32_t* new_tables, int32_t* new_lens,
                              int32_t* gather_idx, int32_t* gather_count,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* Ids of valid pages in ascending physical order (the order of the
 * reference's get_layer_kv, kessie_hip_kernels.py:558-564) into out_idx,
 * their number into *out_count. */
int kessie_page_valid_list(const int8_t* page_valid, int num_pages,
                           int32_t* out_idx, int32_t* out_count,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* Byte copy of whole pages: dst[i] = src_pool[idx[i]] for i < n, each page
 * `page_bytes` long (multiple of 16, 16-byte aligned pointers).  When
 * count_dev is non-NULL the number of pages copied is min(n, *count_dev)
 * read on the device (n is then the capacity of dst and idx).  Pages whose
 * id lies outside [0,num_pages) are skipped (dst[i] is left untouched). */
int kessie_page_gather(const void* src_pool, int64_t page_bytes,
                       const int32_t* idx, const int32_t* count_dev, int n,
                       int num_pages, void* dst, void* stream);

/* =========================================================================
 * Producers around the attention call
 * ========================================================================= */

/* Fog logit bias of the serving path into buf[0:kv_len] (`dtype` elements),
 * replacing _FogCache._compute_into (kessie_attention.py:114-139): with
 * B = int(kv_len * (1.0 - fog_start)) (double arithmetic, as in Python),
 * buf[p] = -fog_alpha * (1 - p/B)^2 for p < B, 0 otherwise, every op rounded
 * to `dtype` as torch's device kernels round it (p/B as p * fp32(1/B)); then
 * buf[r] = dtype(recall_boost) for each recall_positions[r] in [0, kv_len)
 * (num_recall int32 device values; duplicates allowed).  One launch (each
 * workgroup sets the recalled positions of its own range, reading the whole
 * recall list: ~kv_len / 256 * num_recall reads, cheap for recall lists of a
 * few thousand positions); no host synchronisation. */
int kessie_fog_bias_fill(void* buf, int dtype, int kv_len, double fog_alpha,
                         double fog_start, const int32_t* recall_positions,
                         int num_recall, double recall_boost, void* stream);

/* Per-sequence fog logit bias for a batch, as fp32 rows the attention
 * kernels read with fog_bias_bstride = row_stride: row b (b < num_rows)
 * holds, at positions p < seq_lens[b] (device int32, clamped to [0, max_len]),
 * exactly what kessie_fog_bias_fill computes in `dtype` for kv_len =
 * seq_lens[b] (each sequence its own fog boundary
 * B_b = int(seq_lens[b] * (1.0 - fog_start))), widened to fp32; positions
 * from seq_lens[b] to max_len - 1 get 0.  Recalled positions below a row's
 * length get dtype(recall_boost).  One launch, no host synchronisation.
 * (kessie_attention.py:114-139 builds one vector per call, for one kv_len;
 * this is that vector for every sequence of a mixed batch.) */
int kessie_fog_bias_fill_rows(float* out, int64_t row_stride,
                              const int32_t* seq_lens, int num_rows,
                              int max_len, int dtype, double fog_alpha,
                              double fog_start,
                              const int32_t* recall_positions, int num_recall,
                              double recall_boost, void* stream);

/* Fog V weights (fp32) into weights[0:seq_len], replacing
 * kessie_build_fog_weights (kessie_hip_kernels.py:403-413): 1 everywhere;
 * with c = int(seq_len * (1.0 - fog_start)) and fog_alpha > 0,
 * weights[i] = (i * fp32(1/max(c-1,1)))^fog_alpha for i < c, the power taken
 * the way torch's device pow(tensor, scalar) takes it (sqrt for 0.5, products
 * for 2 and 3, powf otherwise). */
int kessie_fog_weights_fill(float* weights, int seq_len, double fog_alpha,
                            double fog_start, void* stream);

/* Slot-mapped write of new K/V rows into the paged cache (the write a
 * serving backend performs before attention): for token t < num_tokens with
 * slot = slot_mapping[t] >= 0 and slot / page_size < num_pages, copies
 * key[t][h][:] and value[t][h][:] (source strides in elements; innermost
 * dimension contiguous) to page slot/page_size, offset slot%page_size of the
 * pool.  Negative slots (padding) are skipped. */
int kessie_kv_cache_write(void* kv_pool, int64_t page_stride,
                          int64_t tok_stride, int64_t kv_stride,
                          int64_t head_stride, const void* key,
                          int64_t key_tok_stride, int64_t key_head_stride,
                          const void* value, int64_t value_tok_stride,
                          int64_t value_head_stride,
                          const int64_t* slot_mapping, int num_tokens,
                          int num_kv_heads, int head_dim, int page_size,
                          int num_pages, int dtype, void* stream);

/* Fog weights of the HF tiered cache (KeSSieCache._compute_fog_mask,
 * kessie_exp3.py:415-425) into weights[0:seq_len] (fp32): with
 * cc = max(1, int(seq_len * fog_start)) and fc = seq_len - cc,
 * w[p] = max((p * fp32(1/max(fc-1,1)))^fog_alpha, 0.01) for p < fc and 1
 * otherwise (all ones when fc <= 0 or fog_alpha <= 0). */
int kessie_hf_fog_weights_fill(float* weights, int seq_len, double fog_alpha,
                               double fog_start, void* stream);

/* out[b][h][t][:] = dtype(fp32(v[b][h][t][:]) * w[t]) with the weights
 * above over seq_len positions (KeSSieCache.update's fog step,
 * kessie_exp3.py:443-445), in one pass; strides in elements, head_dim
 * contiguous, 16-byte aligned rows. */
int kessie_hf_fog_apply(const void* v, int64_t v_batch_stride,
                        int64_t v_head_stride, int64_t v_tok_stride, void* out,
                        int64_t out_batch_stride, int64_t out_head_stride,
                        int64_t out_tok_stride, int batch, int num_heads,
                        int seq_len, int head_dim, double fog_alpha,
                        double fog_start, int dtype, void* stream);

/* KeSSieCache.update for one layer in one launch (kessie_exp3.py:427-445:
 * the torch.cat append of key/value_states, then the fog step): new_k/new_v
 * [B][H][t_new][D] are written into the K/V arenas at window positions
 * n_old .. n_old+t_new-1 (k_arena/v_arena point at the window start and share
 * the arena strides), and, when vfog is non-null, vfog[b][h][t] =
 * dtype(fp32(V[t]) * w[t]) over all n_old + t_new window tokens with the
 * weights of kessie_hf_fog_weights_fill (V[t] read from the arena for
 * t < n_old and from new_v otherwise).  Strides in elements, head_dim
 * contiguous, 16-byte aligned rows (else KESSIE_ERR_UNSUPPORTED, nothing
 * launched). */
int kessie_hf_append_fog(void* k_arena, void* v_arena, int64_t arena_batch_stride,
                         int64_t arena_head_stride, int64_t arena_tok_stride,
                         const void* new_k, int64_t k_batch_stride,
                         int64_t k_head_stride, int64_t k_tok_stride,
                         const void* new_v, int64_t v_batch_stride,
                         int64_t v_head_stride, int64_t v_tok_stride,
                         void* vfog, int64_t vfog_batch_stride,
                         int64_t vfog_head_stride, int64_t vfog_tok_stride,
                         int batch, int num_heads, int n_old, int t_new,
                         int head_dim, double fog_alpha, double fog_start,
                         int dtype, void* stream);

/* =========================================================================
 * Semantic index query
 * ========================================================================= */

/* Workspace bytes for kessie_index_query (0 when top_k == 0). */
size_t kessie_index_query_workspace_bytes(int num_chunks, int top_k);

/* Cosine similarity of query_embed (fp32 [embed_dim]) against every row of
 * index_embeds ([num_chunks][row_stride] elements of `dtype`, 16-byte aligned
 * rows, embed_dim <= 1024): sim_i = dot(q, e_i) * inv(|q|) * inv(|e_i|) with
 * fp32 accumulation, into similarities[num_chunks].  norm_mode picks the
 * normalisation of the search being replaced: 0 = 1/sqrt(n^2+1e-8)
 * (_kessie_index_query_kernel, kessie_hip_kernels.py:344-360), 1 =
 * 1/(n+1e-8) (the numpy searches, kessie_exp3.py:1866-1869), 2 = 1/n with
 * norms below 1e-8 taken as 1 (VectorIndex, kessie_exp3.py:74-76,89-105).
 * Then, when top_k > 0 (<= 1024), the top_k rows ordered by similarity
 * descending, ties by ascending row index, into top_ids / top_scores (either
 * may be NULL); entries past num_chunks are -1 / -inf. */
int kessie_index_query(const void* index_embeds, int64_t row_stride,
                       int num_chunks, int embed_dim, int dtype,
                       int norm_mode, const float* query_embed,
                       float* similarities,
                       int top_k, int32_t* top_ids, float* top_scores,
                       void* workspace, size_t workspace_bytes, void* stream);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* KESSIE_MI355X_H */
