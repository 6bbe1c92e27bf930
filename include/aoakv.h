/*
 * aoakv.h -- C ABI of libaoakv.so, the MI355X (gfx950) implementation of
 * AOA-KV's single-layer decode hot path.
 *
 * The entry points replace the ops of the reference's pybind module
 * `quest._kernels` (kernels/aoa_kv/quest/ops/csrc/bsk_ops.cu:4-20,
 * bsk_ops.h:23-126), one for one, with the same argument meaning:
 *
 *   append_kv_cache_prefill      -> aoakv_append_kv_cache_prefill
 *   append_kv_cache_decode       -> aoakv_append_kv_cache_decode
 *   estimate_attn_score          -> aoakv_estimate_attn_score
 *   topk_filtering               -> aoakv_topk_filtering
 *   BatchDecodeWithPagedKVCache  -> aoakv_decode_workspace_size,
 *     PyTorchWrapper                aoakv_workspace_init,
 *     .begin/forward/end_forward    aoakv_decode_sparse_attn
 *   prefill_with_paged_kv_cache  -> aoakv_prefill_with_paged_kv_cache
 *   apply_rope_in_place          -> aoakv_apply_rope_in_place
 *   rms_norm_forward             -> aoakv_rms_norm_forward
 *
 * plus fused entry points: aoakv_sparse_decode_layer (estimate + top-k +
 * sparse decode for one layer), aoakv_estimate_topk, and
 * aoakv_rope_append_kv_cache_decode (RoPE + decode append).
 *
 * Conventions
 *   - All tensor arguments are device pointers (plain pointers, no torch
 *     types).  fp16 data is passed as `void*` and holds IEEE binary16.
 *   - Paged cache of one layer (reference kv_cache.py:19-23):
 *       layout NHD (0): [max_pages, 2, page_size, num_heads, head_dim]
 *       layout HND (1): [max_pages, 2, num_heads, page_size, head_dim]
 *     slot 0 = K, slot 1 = V.  The metadata cache uses the same layout with
 *     "tokens" = kv pages: slot 0 = per-page Kmax, slot 1 = per-page Kmin
 *     (reference decode_page.cuh:425-449).
 *   - v_log_norm: [max_pages, num_kv_heads] fp16, indexed by PHYSICAL kv page
 *     (reference controller.py:43-47).  v_mean: [max_pages, num_kv_heads,
 *     head_dim] fp16, the simulation's per-page mean of V
 *     (filter_util.py:797-834), which the decode append needs for its
 *     running mean (filter_util.py:669-716).
 *   - Page tables: kv_indptr[B+1], kv_indices[], kv_last_page_len[B] and
 *     metadata_indptr[B+1], metadata_indices[] are int32 device arrays
 *     (reference paged_kv_t, decode_page.cuh:79-352).
 *   - Semantics are the reference simulation's (filter_util.py:269-407,
 *     quest_attention.py:196-382): every page, including the partial last
 *     one, is scored; fixed selection forces the first and last page;
 *     k = min(max(3, min(L, budget) / page_size), P); scores are fp32.
 *     AOAKV_FLAG_QUEST_KERNEL selects the reference kernel's convention
 *     instead (see there).
 *   - Every call is asynchronous on `stream` (a hipStream_t), allocates no
 *     device memory and performs no host synchronisation.
 *   - Return value: 0 on success, otherwise an AOAKV_ERR_* code;
 *     aoakv_last_error() then describes the failure (thread-local).
 *   - Supported shapes: head_dim 64, 128 or 256 (the reference's
 *     SWITCH_HEAD_DIM, decode_page.cuh:718-760), page_size 1..32,
 *     num_heads <= 256, num_qo_heads a multiple of num_kv_heads with group
 *     size 1, 2, 4 or 8.  head_dim 128 with page_size 16 runs the tuned
 *     kernels; the other shapes run simpler kernels with the same results
 *     (AOAKV_FLAG_SINGLE_LAUNCH is then ignored: two launches).
 */
#ifndef AOAKV_H_
#define AOAKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AOAKV_OK 0
#define AOAKV_ERR_INVALID 1     /* bad argument (null pointer, size, budget) */
#define AOAKV_ERR_UNSUPPORTED 2 /* unsupported head_dim / page_size / layout */
#define AOAKV_ERR_HIP 3         /* HIP runtime error (launch failure) */

#define AOAKV_LAYOUT_NHD 0u
#define AOAKV_LAYOUT_HND 1u

/* flags for scoring / selection */
#define AOAKV_FLAG_VALUE_AWARE 1u /* AOA-KV score (else plain Quest bound)   */
#define AOAKV_FLAG_FIXED 2u       /* force first and last page (sim `fixed`) */
/* aoakv_sparse_decode_layer only: run scoring, top-k and decode in ONE launch
 * (scoring workers, per-head top-k and decode items handing over through
 * the workspace) instead of two launches.  A call whose rows exceed 4,096
 * pages, or whose one-launch grid would exceed 16,777,215 workgroups (a
 * dispatch's 32-bit work-item count at 256 per workgroup), runs as the two
 * launches, with the same results.  Workgroups wait on lower-indexed
 * workgroups of the launch, each wait bounded; if one gives up,
 * AOAKV_WS_ERR_WAIT is set in the workspace's error word, the output is
 * invalid and handoff words may be left set.  Every later one-launch call
 * on that workspace then reads no handoff word (its scoring items may still
 * write their score words) and writes NaN outputs until
 * aoakv_workspace_init re-initialises it. */
#define AOAKV_FLAG_SINGLE_LAUNCH 4u
/* The reference KERNEL's selection convention instead of the simulation's
 * (controller.py:113-124, quest/utils/__init__.py:196-246,
 * decode_attn.cuh:297-306): the last page is not scored and is always
 * attended; k = min(max(1, budget / page_size), P) pages are attended, the
 * last one plus the k - 1 best of the others.  Score rows then hold P - 1
 * entries and selection rows the k - 1 chosen pages (the reference's
 * [H, page_budget - 1] top-k output); the decode adds the last page itself.
 * Not combinable with AOAKV_FLAG_FIXED.  The value statistic is still read
 * at the page's own physical index. */
#define AOAKV_FLAG_QUEST_KERNEL 8u
/* aoakv_decode_sparse_attn and aoakv_sparse_decode_layer with grouped query
 * attention (num_qo_heads > num_kv_heads): one decode workgroup per (kv
 * head, chunk of 8 selected pages) loads the chunk's K/V once and serves the
 * kv head's whole query group, as the reference's decode block does with one
 * threadIdx.y per query head (decode_attn.cuh:497-500, 1158-1171).  Without
 * it (the default) every query head has its own workgroups; the query heads
 * of a group then run on one XCD and share the K/V through its L2, with
 * G times the parallelism -- faster on MI355X at the shapes measured
 * (bench.py extra.gqa_32q_8kv_32k).  Same arithmetic per query head either
 * way: the outputs are identical. */
#define AOAKV_FLAG_GROUPED_DECODE 16u

/* The workspace error word: 32-bit word AOAKV_WS_ERR_WORD of a decode
 * workspace (offset 8 bytes), OR-ed by the kernels of every entry point that
 * takes a workspace, zeroed by aoakv_workspace_init.  The library never
 * reads it back on the host (that would synchronise); a caller checks it
 * when it wishes, e.g. once per generated token.
 *   AOAKV_WS_ERR_WAIT       a bounded wait of the one-launch layer gave up
 *                           (see AOAKV_FLAG_SINGLE_LAUNCH)
 *   AOAKV_WS_ERR_TRUNCATED  a sequence's device page table (kv_indptr) held
 *                           more pages than the call was sized for
 *                           (max_pages, score_stride, sel_stride, or a
 *                           kernel limit): that sequence's scores,
 *                           selection and output were computed on its first
 *                           pages only.  No access leaves the sized buffers. */
#define AOAKV_WS_ERR_WORD 2u
/* Bytes of the control words at the start of every workspace (the error
 * word among them); no call needs fewer. */
#define AOAKV_WORKSPACE_CTL_BYTES 256u
#define AOAKV_WS_ERR_WAIT 1u
#define AOAKV_WS_ERR_TRUNCATED 2u

/* Thread-local description of the last failure ("" when none). */
const char* aoakv_last_error(void);

/* Library version string. */
const char* aoakv_version(void);

/*
 * Bulk append of N new tokens of ONE sequence into the paged cache, with
 * metadata maintenance.  Replaces append_kv_cache_prefill
 * (reference bsk_ops.h:53-68, page.cu:107-222, decode_page.cuh:528-692).
 *
 * k, v: [N, num_heads, head_dim] fp16 (NHD, contiguous).  The cache pages
 * must already be reserved: num_kv_pages pages listed in kv_indices (host
 * count), the last one holding kv_last_page_len tokens after the append.
 * metadata_indices lists ceil(num_kv_pages / page_size) metadata pages.
 * For each page touched: K/V stored; Kmax/Kmin folded; on a page that
 * starts empty V̄ = fp16(sum_fp32 / n) (compute_page_v_mean), on a page
 * already holding tokens V̄ follows the running mean of
 * update_mean_filter token by token; log‖V̄‖ stored in v_log_norm.
 */
int aoakv_append_kv_cache_prefill(const void* k, const void* v, uint32_t num_new_tokens,
                                  void* kv_data, const int32_t* kv_indices,
                                  uint32_t num_kv_pages, uint32_t kv_last_page_len,
                                  void* metadata_data, const int32_t* metadata_indices,
                                  void* v_log_norm, void* v_mean, uint32_t num_heads,
                                  uint32_t head_dim, uint32_t page_size, uint32_t layout,
                                  void* stream);

/*
 * Append one token per sequence for a batch of B sequences (decode step).
 * Replaces append_kv_cache_decode (reference bsk_ops.h:70-85, page.cu:6-105,
 * decode_page.cuh:398-506); follows filter_util.py:669-716,758-795.
 *
 * k, v: [B, num_heads, head_dim] fp16.  The slot of the new token must be
 * reserved: kv_last_page_len[b] already counts it.
 */
int aoakv_append_kv_cache_decode(const void* k, const void* v, uint32_t batch_size,
                                 void* kv_data, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                 void* metadata_data, const int32_t* metadata_indptr,
                                 const int32_t* metadata_indices, void* v_log_norm,
                                 void* v_mean, uint32_t num_heads, uint32_t head_dim,
                                 uint32_t page_size, uint32_t layout, void* stream);

/*
 * Rotary position embedding of q [seq_len, num_qo_heads, head_dim] and
 * k [seq_len, num_kv_heads, head_dim] (NHD, fp16), in place; token n is at
 * position past_kv_len + n.  Replaces apply_rope_in_place (reference
 * page.cu:224-265, QKApplyRotaryInPlaceKernel decode_page.cuh:785-869): the
 * Llama rotate-half form with frequency (1/rope_scale) *
 * (1/rope_theta)^(2i/head_dim) for the dim pair (i, i + head_dim/2),
 * computed in fp32, rounded once to fp16.  The reference defaults are
 * rope_scale 1, rope_theta 1e4 (quest/utils/__init__.py:42-45).
 * Positions up to 2^24.
 */
int aoakv_apply_rope_in_place(void* q, void* k, uint32_t seq_len, uint32_t past_kv_len,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              float rope_scale, float rope_theta, void* stream);

/*
 * RMSNorm of x [rows, n] (fp16, row-major) with weight w [n] into out [rows,
 * n]: out = fp16((x * r) * w), r = 1 / sqrt(sum(x^2) / n + epsilon), x and w
 * widened to fp32 and the sum in fp32.  Replaces rms_norm_forward (reference
 * bsk_ops.h:29, rms_norm.cu:76-213, quest/utils/__init__.py:54-67; the
 * reference model's LlamaRMSNorm, quest/models/llama.py:62-72).
 * n a multiple of 8, 8 <= n <= 65536; rows >= 1.  out may alias x.
 */
int aoakv_rms_norm_forward(const void* x, const void* w, void* out, uint32_t rows, uint32_t n,
                           float epsilon, void* stream);

/*
 * The decode step's RoPE and append in one launch: aoakv_apply_rope_in_place
 * on q [B, num_qo_heads, D] and k [B, num_heads, D] at each sequence's new
 * position (the token the page table already counts: L_b - 1), then
 * aoakv_append_kv_cache_decode of the rotated k and v.  Same results, bit
 * for bit, as the two calls; q and k are rotated in place as the reference's
 * QuestAttention.forward leaves them (QuestAttention.py:98-111).
 */
int aoakv_rope_append_kv_cache_decode(void* q, void* k, const void* v, uint32_t batch_size,
                                      uint32_t num_qo_heads, void* kv_data,
                                      const int32_t* kv_indptr, const int32_t* kv_indices,
                                      const int32_t* kv_last_page_len, void* metadata_data,
                                      const int32_t* metadata_indptr,
                                      const int32_t* metadata_indices, void* v_log_norm,
                                      void* v_mean, uint32_t num_heads, uint32_t head_dim,
                                      uint32_t page_size, uint32_t layout, float rope_scale,
                                      float rope_theta, void* stream);

/*
 * Page scores of every page of every sequence.  Replaces estimate_attn_score
 * (reference bsk_ops.h:41-51, estimate.cu:6-90, decode_attn.cuh:145-199,
 * 276-443); follows filter_util.py:269-380,968-1018:
 *   bound(p) = sum_d max(q_d*Kmax_d, q_d*Kmin_d)                       (fp32)
 *   value-aware: 2*bound/sqrt(d) [logsumexp over a GQA group]
 *                + 2*log‖V̄_p‖                                          (fp32)
 *   plain Quest: bound [summed over a GQA group]
 *
 * q: [B, num_qo_heads, head_dim] fp16.  scores: [B, num_kv_heads,
 * score_stride] fp32, entry p < P_b written (p < P_b - 1 with
 * AOAKV_FLAG_QUEST_KERNEL).  max_pages >= every P_b.
 */
int aoakv_estimate_attn_score(const void* q, float* scores, uint32_t score_stride,
                              const void* metadata_data, const int32_t* metadata_indptr,
                              const int32_t* metadata_indices, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              const void* v_log_norm, uint32_t batch_size, uint32_t max_pages,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              uint32_t page_size, uint32_t layout, uint32_t flags, void* stream);

/*
 * Per-(sequence, kv head) top-k pages under a token budget.  Replaces
 * topk_filtering (reference bsk_ops.h:34-39, topk.cu:7-46,
 * decode_select_k.cuh:26-61); follows filter_util.py:373-380.
 *
 * k_b = min(max(3, min(L_b, budget_b) / page_size), P_b) where budget_b is
 * token_budgets[b] when token_budgets != NULL, else token_budget.  With
 * AOAKV_FLAG_FIXED pages 0 and P_b-1 are always selected.  Ties are broken
 * towards the lower page index.  Output: sel_pages[B, num_kv_heads,
 * sel_stride] int32 PHYSICAL page ids (kv_indices entries) of the selected
 * pages in ascending logical order; entries >= k_b untouched.
 * sel_stride >= max_b k_b.  A score row is the candidate set: at most
 * score_stride <= 16384 pages (16383 with AOAKV_FLAG_QUEST_KERNEL) per
 * (sequence, head) take part, as the reference's top-k over an [H, n] row.
 * error_word: NULL, or a device word into which a sequence whose page table
 * holds more pages than a score row (or than 16384) ORs
 * AOAKV_WS_ERR_TRUNCATED (its selection is made from the row's pages, as
 * above); the word is only ever set, the caller clears it.  A workspace's
 * error word (byte offset 8 of a workspace, AOAKV_WS_ERR_WORD) may be
 * passed.  With AOAKV_FLAG_QUEST_KERNEL: k_b - 1 pages chosen among the
 * first P_b - 1 (score rows of P_b - 1 entries), the last page not written.
 */
int aoakv_topk_filtering(const float* scores, uint32_t score_stride,
                         const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, uint32_t token_budget,
                         const int32_t* token_budgets, int32_t* sel_pages, uint32_t sel_stride,
                         uint32_t batch_size, uint32_t num_kv_heads, uint32_t page_size,
                         uint32_t flags, uint32_t* error_word, void* stream);

/*
 * Bytes of the caller-owned workspace for aoakv_decode_sparse_attn and
 * aoakv_sparse_decode_layer (replaces the buffers BatchDecodeHandler
 * allocates in begin_forward, reference decode_handler.cuh:73-136).
 * max_sel_pages: upper bound on pages attended per (sequence, head).  The
 * decode splits a head's pages into chunks of 8 whose partials (head_dim + 4
 * floats each) are merged through the workspace; with head_dim 128 and
 * page_size 16 (the tuned kernels) at most 8192 pages per head, with the
 * other shapes any number.
 */
size_t aoakv_decode_workspace_size(uint32_t batch_size, uint32_t num_qo_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim,
                                   uint32_t max_sel_pages);

/*
 * Workspace bytes for aoakv_sparse_decode_layer with AOAKV_FLAG_SINGLE_LAUNCH
 * at its fastest: the decode workspace plus one word per (sequence, query
 * head, page) through which the launch's scoring items hand their scores to
 * its top-k (polled directly, no arrival counter; with GQA a copy per query
 * head, which that head's decode items read and clear).  A workspace of only
 * aoakv_decode_workspace_size bytes still works (counter handoff).  No
 * counterpart in the reference (its decode handler sizes its own buffers,
 * decode_handler.cuh:73-136).
 */
size_t aoakv_layer_workspace_size(uint32_t batch_size, uint32_t num_qo_heads,
                                  uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t max_sel_pages, uint32_t max_pages);

/*
 * Zero the workspace's arrival counters.  Call once after allocating a
 * workspace (the kernels leave the counters at zero on exit).
 */
int aoakv_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sparse decode attention over selected pages, split-K over pages with an
 * in-kernel merge.  Replaces BatchDecodeWithPagedKVCachePyTorchWrapper
 * .forward (reference approx_attn.cu:68-151, decode_attn.cuh:482-688,
 * 1004-1044); follows quest_attention.py:265-268,347-356 (fp16-rounded
 * logits, fp32 softmax, fp16 output).
 *
 * q, o: [B, num_qo_heads, head_dim] fp16.  sel_pages as written by
 * aoakv_topk_filtering (physical ids, per kv head, sel_stride); the number
 * of pages per (b, head) is recomputed from the same k rule.  sel_pages ==
 * NULL attends every page (dense decode).  flags: AOAKV_FLAG_QUEST_KERNEL
 * (the rows hold the k - 1 pages besides the last page, which is attended
 * as well, as BatchDecodeWithPagedKVCacheKernel does with kv_last_page_idx)
 * or 0.
 */
int aoakv_decode_sparse_attn(const void* q, void* o, const void* kv_data,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* kv_last_page_len, const int32_t* sel_pages,
                             uint32_t sel_stride, uint32_t token_budget,
                             const int32_t* token_budgets, void* workspace,
                             size_t workspace_bytes, uint32_t batch_size, uint32_t max_pages,
                             uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                             uint32_t page_size, uint32_t layout, uint32_t flags, void* stream);

/*
 * One decode layer: estimate + top-k (fused, last-arriving workgroup per
 * head selects) then sparse decode (fused merge).  Equivalent to the three
 * calls above; scores and sel_pages are written as they would be.
 * Reference call sequence: QuestAttention.py:135-157.
 */
int aoakv_sparse_decode_layer(const void* q, void* o, const void* kv_data,
                              const int32_t* kv_indptr, const int32_t* kv_indices,
                              const int32_t* kv_last_page_len, const void* metadata_data,
                              const int32_t* metadata_indptr, const int32_t* metadata_indices,
                              const void* v_log_norm, float* scores, uint32_t score_stride,
                              int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                              const int32_t* token_budgets, void* workspace,
                              size_t workspace_bytes, uint32_t batch_size, uint32_t max_pages,
                              uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim,
                              uint32_t page_size, uint32_t layout, uint32_t flags, void* stream);

/*
 * aoakv_sparse_decode_layer without a workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, results and bits as aoakv_sparse_decode_layer's
 * two-launch path (AOAKV_FLAG_SINGLE_LAUNCH is rejected); its workspace is
 * a 16 MiB device array inside the library, one per GPU, held until the
 * process ends.  A call whose decode workspace
 * (aoakv_decode_workspace_size of the call's shape) exceeds 16 MiB is
 * rejected with AOAKV_ERR_INVALID.  Allocates nothing.  Calls share their
 * GPU's array: two calls that overlap on one GPU (different streams, or
 * different host threads without ordering) race and give wrong results.
 * The array has an error word like a workspace's (AOAKV_WS_ERR_TRUNCATED
 * when a device page table is longer than max_pages; the sequence is cut
 * safely, as in aoakv_sparse_decode_layer): aoakv_noalloc_error reads and
 * clears it.  The array's device address is looked up on the first call on
 * a device (hipGetSymbolAddress); a caller that captures the call into a
 * HIP graph calls aoakv_noalloc_init on that device first, outside capture.
 */
int aoakv_sparse_decode_layer_noalloc(
    const void* q, void* o, const void* kv_data, const int32_t* kv_indptr,
    const int32_t* kv_indices, const int32_t* kv_last_page_len, const void* metadata_data,
    const int32_t* metadata_indptr, const int32_t* metadata_indices, const void* v_log_norm,
    float* scores, uint32_t score_stride, int32_t* sel_pages, uint32_t sel_stride,
    uint32_t token_budget, const int32_t* token_budgets, uint32_t batch_size, uint32_t max_pages,
    uint32_t num_qo_heads, uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
    uint32_t layout, uint32_t flags, void* stream);

/*
 * Set-up for aoakv_sparse_decode_layer_noalloc on the current device: looks
 * up the device address of the library's scratch array once (later calls
 * are no-ops).  Call it before capturing a noalloc call into a HIP graph.
 * No counterpart in the reference; for callers that cannot allocate.
 */
int aoakv_noalloc_init(void);

/*
 * Reads the current device's scratch error word (AOAKV_WS_ERR_* bits set by
 * aoakv_sparse_decode_layer_noalloc calls since it was last cleared) after
 * synchronising `stream`, into *error_bits; with clear != 0 a non-zero word
 * is then zeroed on `stream`.  Synchronises, so not for use under capture.
 * No counterpart in the reference; for callers that cannot allocate.
 */
int aoakv_noalloc_error(uint32_t* error_bits, uint32_t clear, void* stream);

/*
 * estimate + top-k in one launch (the first launch of
 * aoakv_sparse_decode_layer): page scores are written to `scores` and the
 * last workgroup of each (sequence, kv head) selects into sel_pages.
 * Equivalent to aoakv_estimate_attn_score followed by aoakv_topk_filtering
 * (reference call sequence QuestAttention.py:135-148).  workspace: as for
 * aoakv_decode_sparse_attn (its arrival counters are used).
 */
int aoakv_estimate_topk(const void* q, const void* metadata_data, const int32_t* metadata_indptr,
                        const int32_t* metadata_indices, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* kv_last_page_len,
                        const void* v_log_norm, float* scores, uint32_t score_stride,
                        int32_t* sel_pages, uint32_t sel_stride, uint32_t token_budget,
                        const int32_t* token_budgets, void* workspace, size_t workspace_bytes,
                        uint32_t batch_size, uint32_t max_pages, uint32_t num_qo_heads,
                        uint32_t num_kv_heads, uint32_t head_dim, uint32_t page_size,
                        uint32_t layout, uint32_t flags, void* stream);

/*
 * Dense causal prefill over the paged cache of ONE sequence.  Replaces
 * prefill_with_paged_kv_cache (reference bsk_ops.h:87-95,
 * batch_prefill.cu:27-117, prefill.cuh:688-1115).
 *
 * q, o: [qo_len, num_qo_heads, head_dim] fp16; the cache holds num_kv_heads
 * heads (num_qo_heads a multiple of it: query head h reads kv head
 * h / (num_qo_heads / num_kv_heads)).  The queries are the last qo_len
 * positions of the L = (num_kv_pages-1)*page_size + kv_last_page_len
 * cached tokens; query i attends keys <= L - qo_len + i when causal.
 * fp16 inputs, fp32 accumulation, fp16 output: on the matrix cores (MFMA)
 * for head_dim 64 / 128 / 256 at page sizes 1, 2, 4, 8, 16 and 32, on a
 * vector kernel for the other page sizes.
 */
int aoakv_prefill_with_paged_kv_cache(const void* q, void* o, const void* kv_data,
                                      const int32_t* kv_indices, uint32_t num_kv_pages,
                                      uint32_t kv_last_page_len, uint32_t qo_len,
                                      uint32_t causal, uint32_t num_qo_heads,
                                      uint32_t num_kv_heads, uint32_t head_dim,
                                      uint32_t page_size, uint32_t layout, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AOAKV_H_ */
