/*
 * std_hip.h — C ABI of libstdhip.so, the MI355X (gfx950) decode hot path of
 * Sparse-to-Dense (STD) speculative decoding.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element
 * counts and strides, and returns an int status:
 *     0            success
 *     < 0          argument validation error (STD_E_*), nothing was launched
 *     > 0          hipError_t reported by the HIP runtime at launch
 * Calls are stream-ordered and asynchronous on `stream` (a hipStream_t passed
 * as void*; NULL is the default stream). No call allocates or frees device
 * memory: scratch space is a caller-owned workspace whose size is queried up
 * front with the matching *_workspace_bytes() function; its contents need no
 * initialisation, and calls that can run concurrently need distinct
 * workspaces. No call synchronizes the device. Apart from
 * std_gqa_decode_noalloc (its own device scratch array per GPU and the
 * lock-guarded table of those arrays' addresses) the library keeps no mutable
 * global state, so distinct streams may be driven from distinct host threads.
 *
 * Layouts (batch size 1, as in the reference):
 *   query     [n_q][q_len][d]         row stride d, head stride q_len*d
 *   KV cache  [n_kv][capacity][d]     row stride d, head stride given per call
 *             (the reference's per-layer view of a [2L,1,Hkv,max_len,D]
 *             tensor has head stride max_len*D: read in place, no copy)
 *   output    [n_q][q_len][d]
 * Query head h reads KV head h / (n_q / n_kv)  (repeat_kv / enable_gqa order).
 * Supported: d == 128, 1 <= n_q/n_kv <= 16, dtype STD_F32, STD_BF16 or STD_F16
 * (fp16 as the reference loads its model, scripts/benchmark_std.py:66; the
 * bf16 and fp16 kernels are the same but for the MFMA element type and the
 * rounding of probabilities and outputs). Exceptions are noted per call.
 */
#ifndef STD_HIP_H
#define STD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
enum { STD_F32 = 0, STD_BF16 = 1, STD_F16 = 2 };

/* validation errors (negative) */
enum {
  STD_OK = 0,
  STD_E_NULL = -1,        /* a required pointer is NULL */
  STD_E_DTYPE = -2,       /* unsupported dtype */
  STD_E_SHAPE = -3,       /* unsupported or inconsistent sizes */
  STD_E_WORKSPACE = -4,   /* workspace smaller than *_workspace_bytes() */
  STD_E_ALIGN = -5,       /* pointer or stride misaligned for 16-byte access */
  STD_E_RANGE = -6        /* length or index past the cache capacity */
};

/* Device status word. The device-length entry points (std_kv_append,
 * std_rope_append, std_qkv_rope_append, std_attn_devlen,
 * std_gqa_decode_indexed with a device length, std_verify_attn_collect_ex
 * with a device length) take an optional int32_t* status in device memory.
 * Where the device length places a row, or the attended keys, past the cache
 * capacity, the kernel leaves that memory alone (rows past the capacity are
 * not written; an attention with an out-of-range length reads nothing and
 * writes NaN outputs) and ORs STD_STATUS_CACHE_OVERFLOW into *status, so
 * that a step replayed from a graph reports it with its next readback (the
 * reference's KVCache.cat raises instead, kv_cache.py:54-69). The word is
 * never cleared by the library. */
enum { STD_STATUS_CACHE_OVERFLOW = 1 };

/* Human-readable text for a status code (static storage). */
const char* std_status_string(int status);

/* Library version, e.g. 0x000100 for 0.1.0. */
int std_version(void);

/* ------------------------------------------------------------------------
 * Draft / autoregressive GQA decode attention (q_len == 1, no mask).
 *
 * Replaces fused_gqa_attention(query, key, value)
 *   (src/std_repro/triton_attention.py:83-112) and the draft dispatch to
 *   F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
 *   (src/std_repro/std_qwen25vl.py:399-417).
 * out[h][:] = sum_j softmax_j(q[h].k[g(h)][j] * scale) v[g(h)][j], j < kv_len.
 * K and V are read in place through their head strides (elements); the
 * reference's .contiguous() copy (std_qwen25vl.py:403-408) is not needed.
 * ------------------------------------------------------------------------ */
size_t std_gqa_decode_workspace_bytes(int n_q, int n_kv, int kv_len, int d);

/* Planning query (host only, no counterpart in the reference): the number of
 * key-range splits per problem that an attention launch over n_problems
 * independent (KV head x batch) problems of `rows` query rows each
 * ((n_q / n_kv) * q_len, 1..96) and kv_len keys uses; one split means no
 * merge launch and no workspace. STD_E_SHAPE / STD_E_DTYPE on bad input. */
int std_attn_split_count(int n_problems, int rows, int kv_len, int dtype);

int std_gqa_decode(const void* q, const void* k, const void* v, void* out,
                   int n_q, int n_kv, int kv_len, int d,
                   long long k_head_stride, long long v_head_stride,
                   float scale, int dtype,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free decode: no counterpart in the reference. For callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc) and cannot keep a workspace either. Same arguments,
 * kernels and results as std_gqa_decode, bit for bit, but the split partials
 * live in a device array of the library (2 MiB + 64 KiB per GPU, held until
 * the process ends; looked up on the first call on each device, which must be
 * the current device and the stream's device). Returns STD_E_WORKSPACE where
 * std_gqa_decode_workspace_bytes() exceeds that size (bf16, fp16: never; fp32: more
 * than 8 query heads per KV head at long kv_len). Calls that overlap on one
 * GPU share the array and race: serialise them (one stream per GPU).
 * Allocates nothing and keeps no other state. */
int std_gqa_decode_noalloc(const void* q, const void* k, const void* v, void* out,
                           int n_q, int n_kv, int kv_len, int d,
                           long long k_head_stride, long long v_head_stride,
                           float scale, int dtype, void* stream);

/* Batched decode: n_batch independent single-query problems of the same
 * shape in one launch (plus one merge launch when the problems are split).
 * Problem b reads
 * q + b*q_batch_stride, k + b*k_batch_stride, v + b*v_batch_stride and
 * writes out + b*out_batch_stride (strides in elements; q/out strides
 * >= n_q*d, 16-byte multiples). Each problem equals std_gqa_decode of that
 * problem to fp32 rounding, bit for bit when both get the same split count
 * (with many problems a launch may stream each unsplit; n_batch = 1 always
 * matches).
 * Serves several sequences' draft steps at once (the reference decodes one
 * sequence per call, triton_attention.py:83-112); the same call over the
 * 28 layers of one draft step is the all-layer roofline unit of the draft
 * attention. n_batch <= 65535. */
size_t std_gqa_decode_batched_workspace_bytes(int n_batch, int n_q, int n_kv, int kv_len, int d);

int std_gqa_decode_batched(const void* q, const void* k, const void* v, void* out,
                           int n_batch, int n_q, int n_kv, int kv_len, int d,
                           long long q_batch_stride, long long k_batch_stride,
                           long long v_batch_stride, long long out_batch_stride,
                           long long k_head_stride, long long v_head_stride,
                           float scale, int dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Append + decode in one launch: the single new K/V row (new_k/new_v
 * [n_kv][1][d], head stride new_head_stride) is written to cache row
 * kv_len - 1, then the call attends over kv_len keys exactly as
 * std_gqa_decode. Replaces the draft attention's KVCache.cat followed by the
 * attention call (std_qwen25vl.py:395-417). */
int std_gqa_decode_append(const void* q, void* k_cache, void* v_cache,
                          const void* new_k, const void* new_v, void* out,
                          int n_q, int n_kv, int kv_len, int d,
                          long long k_head_stride, long long v_head_stride,
                          long long new_head_stride, float scale, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Dense verify attention for q_len appended query rows (offset-causal).
 *
 * Replaces the verify forward's attention: repeat_kv + math SDPA with the
 *   additive causal mask (src/specvlm/models/modeling_qwen2_5_vl.py:1096-1132,
 *   mask :65-126 and :1388-1399; backend std_qwen25vl.py:111-116, :802).
 * kv_len counts every cached key including the q_len new rows, which the
 * caller has already appended. Query row i (0-based) sees keys
 * [0, kv_len - q_len + i], the offset_causal_mask of
 * src/std_repro/sparse_verify_spike.py:24-42. Requires 1 <= q_len,
 * q_len * (n_q/n_kv) <= 96 (gamma + 1 <= 13 at 7 query heads per KV head),
 * q_len <= kv_len.
 * ------------------------------------------------------------------------ */
size_t std_verify_attn_workspace_bytes(int n_q, int n_kv, int q_len, int kv_len, int d);

int std_verify_attn(const void* q, const void* k, const void* v, void* out,
                    int n_q, int n_kv, int q_len, int kv_len, int d,
                    long long k_head_stride, long long v_head_stride,
                    float scale, int dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Append + verify in one launch: the q_len new K/V rows (new_k/new_v
 * [n_kv][q_len][d], strides in elements) are written to cache rows
 * [kv_len - q_len, kv_len), then the call attends exactly as std_verify_attn.
 * Replaces the verify forward's KVCache.cat followed by its attention
 * (modeling_qwen2_5_vl.py:1057-1132). Workspace: std_verify_attn_workspace_bytes. */
int std_verify_attn_append(const void* q, void* k_cache, void* v_cache,
                           const void* new_k, const void* new_v, void* out,
                           int n_q, int n_kv, int q_len, int kv_len, int d,
                           long long k_head_stride, long long v_head_stride,
                           long long new_head_stride, long long new_row_stride,
                           float scale, int dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Text-to-video top-K selection for one layer.
 *
 * Replaces the selection prefill's probability materialisation
 *   (modeling_qwen2_5_vl.py:966-995 via :1115-1123) plus
 *   build_sparse_selection (src/std_repro/std_qwen25vl.py:175-231).
 * q_text  [n_q][text_len][d]: the text-suffix query rows (RoPE applied), row
 *         i at absolute position text_start + i; text_len = prompt_len -
 *         text_start.
 * k       [n_kv][capacity][d] with head stride k_head_stride, keys
 *         [0, prompt_len) valid.
 * score[g][j] = sum over the n_q/n_kv query heads h of group g and text rows
 *   i with j <= text_start + i of softmax_i(q[h][i].k[g][:] * scale)[j],
 *   the causal text-row softmax over keys [0, text_start + i]. Logits, exp
 *   and sums are computed in fp64 from the exact input values.
 * visual_pos [n_visual] int32, strictly increasing absolute positions < prompt_len.
 * topk_out [n_kv][k] int32: for every KV head the k visual positions with the
 *   largest score (ties go to the lowest position), sorted ascending.
 * scores_out (optional, may be NULL) [n_kv][prompt_len] fp64 column scores.
 * ------------------------------------------------------------------------ */
size_t std_select_topk_workspace_bytes(int n_q, int n_kv, int text_len, int prompt_len,
                                       int n_visual, int d);

int std_select_topk(const void* q_text, const void* k,
                    int n_q, int n_kv, int text_len, int prompt_len, int text_start, int d,
                    long long k_head_stride, int dtype,
                    const int32_t* visual_pos, int n_visual, int k_select,
                    int32_t* topk_out, double* scores_out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Selection from materialised attention probabilities: the reference's own
 * input. Replaces build_sparse_selection(attentions, ...) per layer
 * (src/std_repro/std_qwen25vl.py:175-231): probs [n_q][text_len][prompt_len]
 * (one layer's [1, n_q, T, P] probabilities of the text suffix's rows,
 * head stride and row stride in elements, columns contiguous; STD_F16, the
 * reference's dtype, STD_BF16 or STD_F32), summed over the query heads of
 * each KV head and the text rows, then the top k_select of the visual
 * columns visual_pos[n_visual] per KV head -> topk_out int32
 * [n_kv][k_select], ascending; ties go to the lowest position. The sums are
 * fp64 (exact for fp16 probabilities); scores_out (optional, fp64
 * [n_kv][prompt_len]) receives them. Any prompt length and strides (the
 * reference's contiguous tensor has row stride P); rows aligned to four
 * elements are read four columns at a time, others element by element. */
size_t std_select_topk_probs_workspace_bytes(int n_q, int n_kv, int text_len, int prompt_len, int n_visual);

int std_select_topk_probs(const void* probs, long long head_stride, long long row_stride, int dtype,
                          int n_q, int n_kv, int text_len, int prompt_len,
                          const int32_t* visual_pos, int n_visual, int k_select,
                          int32_t* topk_out, double* scores_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Compact-index construction: per KV head, the sorted union of the
 * non-visual positions and that head's top-K visual positions
 *   (std_qwen25vl.py:286-291: torch.unique(cat([non_visual, topk[h]]))).
 * The two sets must be disjoint and each sorted ascending.
 * idx_out [n_kv][n_nonvisual + k] int32.
 * ------------------------------------------------------------------------ */
int std_build_compact_index(const int32_t* non_visual, int n_nonvisual,
                            const int32_t* topk, int k_select, int n_kv,
                            int32_t* idx_out, void* stream);

/* ------------------------------------------------------------------------
 * Sparse-cache compaction gather for one layer, K and V together.
 *
 * Replaces copy_prompt_cache + compact_sparse_prompt_cache
 *   (std_qwen25vl.py:265-320): sparse[g][s][:] = dense[g][idx[g][s]][:] for
 *   s < compact_len, read straight from the dense cache (no full-prompt copy).
 * Indices >= dense_rows are rejected with STD_E_RANGE only when checked on the
 * host; the kernel itself skips any out-of-range index.
 * ------------------------------------------------------------------------ */
int std_compact_kv(const void* dense_k, const void* dense_v, void* sparse_k, void* sparse_v,
                   const int32_t* idx, int n_kv, int compact_len, int d,
                   long long dense_head_stride, int dense_rows,
                   long long sparse_head_stride, int sparse_rows,
                   int dtype, void* stream);

/* ------------------------------------------------------------------------
 * KV append at a device-resident length.
 *
 * Replaces KVCache.cat (src/specvlm/kv_cache/kv_cache.py:54-69) without the
 * CPU-resident length: rows are written at positions *len_dev + r,
 * r < rows. new_k/new_v are [n_kv][rows][d] with head stride new_head_stride
 * and row stride new_row_stride (elements; the projection output viewed as
 * [1, Hkv, q_len, D] has head stride D and row stride Hkv*D). Writes at or
 * past `capacity` are skipped. The length itself is advanced separately with
 * std_len_add so that every layer of a step appends at the same position.
 * ------------------------------------------------------------------------ */
int std_kv_append(void* cache_k, void* cache_v, const void* new_k, const void* new_v,
                  int n_kv, int rows, int d,
                  long long cache_head_stride, long long new_head_stride, long long new_row_stride,
                  int capacity, const int32_t* len_dev, int dtype, int32_t* status, void* stream);

/* len[i] += delta for i < n (device int32). */
int std_len_add(int32_t* len_dev, int n, int delta, void* stream);

/* ------------------------------------------------------------------------
 * Rotary embedding fused with the K/V cache append, at a device length and a
 * device position (the decode-step glue that keeps lengths and positions on
 * the GPU, so a whole decode step can be captured in a HIP graph).
 *
 * Replaces, for the decode and verify rows, apply_multimodal_rotary_pos_emb
 *   (modeling_qwen2_5_vl.py:690-732; with three identical position rows the
 *   multimodal embedding is the 1-D rotate-half embedding), the q/k/v
 *   transposes and KVCache.cat (src/specvlm/kv_cache/kv_cache.py:54-69).
 * qkv is the fused projection output [n_rows][(n_q + 2 n_kv) d] (row stride
 * qkv_row_stride elements): query heads, then key heads, then value heads.
 * Row r has position *pos_dev + pos_offset + r; angle = float(pos) *
 * inv_freq[j] (fp32 table of d/2 entries), cos/sin rounded to the dtype, and
 * x * cos + rotate_half(x) * sin evaluated op by op with dtype rounding (as
 * torch evaluates it). Rotated queries go to q_out [n_q][n_rows][d]; rotated
 * keys and the values go to cache row *len_dev + r (head stride
 * cache_head_stride); rows at or past `capacity` are not written. The length
 * is not advanced (std_len_add does that once per step).
 * ------------------------------------------------------------------------ */
int std_rope_append(const void* qkv, long long qkv_row_stride, void* q_out, void* cache_k, void* cache_v,
                    int n_rows, int n_q, int n_kv, int d, long long cache_head_stride, int capacity,
                    const int32_t* len_dev, const int32_t* pos_dev, int pos_offset,
                    const float* inv_freq, int dtype, int32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Offset-causal GQA attention at a device length (decode when q_len == 1).
 *
 * Replaces, for graph-captured decode steps, the dense verify attention
 *   (modeling_qwen2_5_vl.py:1007-1140, mask :65-126) and the sparse draft
 *   attention (std_qwen25vl.py:399-431) with the cache length read on the
 *   device: the cache holds *len_dev + q_len valid rows (the last q_len written
 *   for this step, e.g. by std_rope_append) and query row i sees keys
 *   [0, *len_dev + i]. The split plan and workspace are those of
 *   std_verify_attn at kv_len = max_kv_len (size the workspace with
 *   std_verify_attn_workspace_bytes(n_q, n_kv, q_len, max_kv_len, d)); a device
 *   length outside [0, max_kv_len - q_len] reads nothing and yields NaN outputs.
 * ------------------------------------------------------------------------ */
int std_attn_devlen(const void* q, const void* k_cache, const void* v_cache, void* out,
                    int n_q, int n_kv, int q_len, const int32_t* len_dev, int max_kv_len, int d,
                    long long k_head_stride, long long v_head_stride, float scale, int dtype,
                    void* workspace, size_t workspace_bytes, int32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Sparse draft decode with index-addressed prompt keys (no compaction copy).
 *
 * Replaces compact_sparse_prompt_cache (std_qwen25vl.py:265-298: the gather of
 * each head's sorted non-visual + top-k prompt rows into the sparse cache)
 * together with the draft's fused_gqa_attention call on that cache
 * (triton_attention.py:83-112 via std_qwen25vl.py:399-431): key j < n_index
 * of KV head g is row index[g * index_head_stride + j] of the dense cache
 * (dense_k / dense_v, dense_rows rows per head; an index outside
 * [0, dense_rows) is clamped); keys n_index <= j < the key count are rows j
 * of k_cache / v_cache (the sparse cache: the draft's own appended rows; its
 * first n_index rows are never read). A selection refresh then rewrites
 * n_index integers per head instead of copying rows.
 *
 * len_dev == NULL: kv_len keys. Otherwise the key count is *len_dev + 1 (this
 * step's row last, as std_attn_devlen with q_len = 1) and kv_len is the
 * maximum the launch is planned for. Single query row per head, bf16 or fp16. index:
 * int32, 16-byte aligned, index_head_stride >= n_index rounded up to 16 (the
 * row is read 16 entries at a time). Workspace:
 * std_gqa_decode_workspace_bytes(n_q, n_kv, kv_len, d).
 * ------------------------------------------------------------------------ */
int std_gqa_decode_indexed(const void* q, const void* dense_k, const void* dense_v, int dense_rows,
                           long long dense_k_head_stride, long long dense_v_head_stride,
                           const int32_t* index, long long index_head_stride, int n_index,
                           const void* k_cache, const void* v_cache, long long k_head_stride,
                           long long v_head_stride, void* out, int n_q, int n_kv, int kv_len,
                           const int32_t* len_dev, int d, float scale, int dtype, void* workspace,
                           size_t workspace_bytes, int32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Greedy acceptance plus cache rollback on the device.
 *
 * Replaces the verify tail of std_generate_qwen25vl
 *   (std_qwen25vl.py:806-815 and the rollback :923-928); the pure contract is
 *   greedy_prefix (src/std_repro/hsd_spike.py:30-43).
 * logits [q_rows][vocab] (row stride logits_row_stride elements).
 * pred[r] = argmax(logits[r]) (first maximum; NaN counts as the maximum).
 * predictions = pred                       if has_pending (q_rows == n_draft+1)
 *             = [*dense_next] ++ pred      otherwise      (q_rows == n_draft)
 * accept = longest prefix with draft[i] == predictions[i]; bonus = predictions[accept].
 * out[0] = accept, out[1] = bonus, out[2 .. 2+n_draft] = predictions.
 * Rollback: rollback_lens is a device int32 array of n_lens cache lengths
 * (e.g. {dense_len, sparse_len}); each is decreased by (n_draft - accept),
 * undoing the rejected draft rows appended to the dense cache by verify and
 * to the sparse cache by drafting. n_lens may be 0.
 * dense_next may be NULL when has_pending != 0.
 * ------------------------------------------------------------------------ */
size_t std_greedy_accept_workspace_bytes(int q_rows, int vocab);

/* ------------------------------------------------------------------------
 * Row argmax as int64 token ids (torch.argmax(logits, -1) semantics: first
 * maximum, NaN counts as the maximum), with no memset and no global
 * semaphore, so a captured HIP graph replays it correctly.
 *
 * Replaces the greedy next-token choice of the decode loops
 *   (std_qwen25vl.py:544, :806 via torch.argmax). logits [rows][vocab] (row
 * stride elements); workspace as std_greedy_accept_workspace_bytes(rows, vocab).
 * ------------------------------------------------------------------------ */
int std_argmax_rows(const void* logits, long long logits_row_stride, int rows, int vocab, int dtype,
                    long long* out, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm, one workgroup per row, graph-capture safe (no global staging):
 * out = weight * dtype(x * rsqrt(mean(x^2) + eps)).
 *
 * Replaces Qwen2RMSNorm.forward (modeling_qwen2_5_vl.py:192-197) in the
 * decode steps; rows have strides x_row_stride / out_row_stride elements.
 * ------------------------------------------------------------------------ */
int std_rms_norm(const void* x, long long x_row_stride, const void* weight, void* out,
                 long long out_row_stride, int rows, int hidden, float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Weight-streaming projection for decode/verify rows (M <= 16), bf16:
 * y[m][n] = sum_k x[m][k] * W[n][k] (+ bias[n]), fp32 accumulation.
 *
 * Replaces, at batch 1, the q/k/v, o, gate/up, down and lm_head projections
 * of the draft, verify and AR steps (torch.nn.functional.linear in the
 * decoder layers of modeling_qwen2_5_vl.py; the per-token GEMVs that A10 of
 * the draft loop spends its time in). W [N][K] row-major (row stride
 * w_row_stride), x [M][K], y [M][N]; K a multiple of 32. One launch;
 * deterministic (K is split over the waves of a workgroup and their partial
 * sums are added in a fixed order). std_gemv_workspace_bytes returns 0 (no
 * workspace is used; the arguments are kept for interface stability).
 * ------------------------------------------------------------------------ */
size_t std_gemv_workspace_bytes(int M, int N, int K);

int std_gemv(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
             const void* bias, void* y, long long y_row_stride, int M, int N, int K, int dtype,
             void* workspace, size_t workspace_bytes, void* stream);

/* The same projection with the decoder's neighbouring elementwise ops in its
 * epilogue (one launch instead of two or three at batch 1):
 *   gated = 0: y = residual + (x W^T + bias)     (residual may be NULL)
 *   gated = 1: W is [2N][K], the gate rows over the up rows (bias, if any,
 *              [2N]); y[m][n] = silu(g) * u with g = (x W^T + b)[m][n] and
 *              u = (x W^T + b)[m][N + n], each rounded to bf16.
 * Every op is rounded to bf16 as torch evaluates it on bf16 tensors:
 * Qwen2MLP's act_fn(gate_proj(x)) * up_proj(x) (modeling_qwen2_5_vl.py:686)
 * and the decoder layer's "hidden_states = residual + hidden_states"
 * (modeling_qwen2_5_vl.py:1215, 1221). residual [M][N] has row stride
 * residual_row_stride; x [M][K]; y [M][N]. gated and residual together are
 * allowed. No workspace.
 */
int std_gemv_ex(const void* x, long long x_row_stride, const void* w, long long w_row_stride,
                const void* bias, const void* residual, long long residual_row_stride, void* y,
                long long y_row_stride, int M, int N, int K, int gated, int dtype, void* stream);

/* std_gemv_ex of one row whose input is a hidden state before its RMSNorm:
 * y = std_gemv_ex(std_rms_norm(x, norm_weight, eps), w, bias, residual,
 * gated) in one launch (one instead of two at batch 1) -- the decoder
 * layer's post_attention_layernorm before the MLP's gate/up projection
 * (modeling_qwen2_5_vl.py:1219-1220) and the final norm before lm_head
 * (modeling_qwen2_5_vl.py:1454, 2122). Every workgroup forms the norm while
 * its first weight stages are in flight (7B gate/up: 43.1 us against 46.5 us
 * for the two launches; lm_head 158.8 against 163.3 us). x, norm_weight [K],
 * K <= 3584 a
 * multiple of 32; y, residual (may be NULL) [N]; x, norm_weight, w 16-byte
 * aligned. The normalised row equals std_rms_norm's bit for bit, and y equals
 * std_rms_norm followed by std_gemv_ex bit for bit where std_gemv_ex streams
 * the weight through its LDS ring (one row, weights of 16 MiB and more: every
 * 7B projection); for smaller weights the K split may differ and elements by
 * one bf16 rounding. No workspace. */
int std_gemv_norm(const void* x, const void* norm_weight, float eps, const void* w, long long w_row_stride,
                  const void* bias, const void* residual, void* y, int N, int K, int gated, int dtype,
                  void* stream);

/* The q|k|v projection of a decode step fused with std_rope_append (one
 * launch instead of two): x [n_rows][K] (n_rows <= 4, K <= 4096, a multiple
 * of 32) times W [(n_q + 2 n_kv) * 128][K] (the q_proj, k_proj, v_proj rows
 * stacked, modeling_qwen2_5_vl.py:778-780, 798-800) plus bias, each output rounded to
 * bf16 as F.linear rounds it, then exactly std_rope_append's rotary embedding
 * and cache append (modeling_qwen2_5_vl.py:690-732, kv_cache.py:54-69): rows
 * at position pos_dev[0] + pos_offset + r, rotated queries to q_out
 * [n_q][n_rows][128], rotated keys and the values to cache row len_dev[0] + r
 * (not written at or past capacity). Outputs equal std_gemv_ex followed by
 * std_rope_append bit for bit when the projection has at least 256 16-column
 * blocks (n_q + 2 n_kv >= 32 heads, as at 7B): std_gemv then splits K over
 * four waves like this launch; for narrower projections it splits K over two
 * waves and elements may differ by one bf16 rounding. With norm_weight (not NULL; one row, K <=
 * 3584) x is the decoder layer's input before its input_layernorm
 * (modeling_qwen2_5_vl.py:1202) and the launch normalises it first, equal to
 * std_rms_norm(x, norm_weight, eps) bit for bit. bf16 only; head_dim 128; the
 * length is not advanced.
 */
int std_qkv_rope_append(const void* x, long long x_row_stride, int n_rows, int K, const void* w,
                        long long w_row_stride, const void* bias, int n_q, int n_kv, int d, void* q_out,
                        void* cache_k, void* cache_v, long long cache_head_stride, int capacity,
                        const int32_t* len_dev, const int32_t* pos_dev, int pos_offset,
                        const float* inv_freq, const void* norm_weight, float eps, int dtype,
                        int32_t* status, void* stream);

int std_greedy_accept(const void* logits, long long logits_row_stride, int q_rows, int vocab,
                      int dtype, const int32_t* draft, int n_draft, int has_pending,
                      const int32_t* dense_next, int32_t* out,
                      int32_t* rollback_lens, int n_lens,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Verify attention with the visual-attention collector riding the same pass.
 *
 * Replaces VerificationCollectorV3._hook (src/std_repro/dynamic_selection.py:
 *   504-519), called from the verify forward at
 *   src/specvlm/models/modeling_qwen2_5_vl.py:1063-1067, together with the
 *   verify attention it rides (std_verify_attn / std_verify_attn_append).
 * out: the verify attention of std_verify_attn; with new_k / new_v (both or
 * neither) the q_len new rows are appended first, as std_verify_attn_append.
 * scores[g][j - vis_begin] (fp32, head stride scores_head_stride) =
 *   sum_i softmax_j( qbar[g][i] . k[g][j] * scale ) over the visual keys
 *   j in [vis_begin, vis_end), where qbar[g][i] is the fp32 mean of the query
 *   rows of KV head g's query heads at position i (the hook's
 *   q.float().reshape(...).mean(dim=2)); i < q_len. Visual keys must be prompt
 *   keys (vis_end <= kv_len - q_len). bf16 or fp16.
 * The collector rows ride the padding rows of the verify's last row tile, so
 * one launch serves (n_q / n_kv + 1) * q <= 80, q <= 16 positions (gamma + 1
 * <= 10 at seven query heads per KV head); out is then std_verify_attn's bit
 * for bit. Longer verifies run in chunks of positions (each chunk reads the
 * cache once more; out within the verify's tolerance, scores summed in the
 * same row order).
 * ------------------------------------------------------------------------ */
size_t std_verify_attn_collect_workspace_bytes(int n_q, int n_kv, int q_len, int kv_len, int d,
                                               int vis_begin, int vis_end);

int std_verify_attn_collect(const void* q, void* k_cache, void* v_cache,
                            const void* new_k, const void* new_v, void* out,
                            int n_q, int n_kv, int q_len, int kv_len, int d,
                            long long k_head_stride, long long v_head_stride,
                            long long new_head_stride, long long new_row_stride,
                            float scale, int dtype, int vis_begin, int vis_end,
                            float* scores, long long scores_head_stride,
                            void* workspace, size_t workspace_bytes, void* stream);

/* The general form (same workspace query, with the visual set's first
 * position and last position + 1 as vis_begin / vis_end):
 *  - any ascending set of visual positions, as the hook gathers
 *    key_states[:, :, visual_positions] (dynamic_selection.py:515):
 *    vis_mask (uint32, at least (vis_end + 31) / 32 words) has bit j % 32 of
 *    word j / 32 set for each visual key j, vis_rank[w] = the number of
 *    visual keys below 32 w, n_visual the set's size; scores[g][r] is the
 *    r-th visual key's. vis_mask == vis_rank == NULL: the whole range
 *    [vis_begin, vis_end) (n_visual = vis_end - vis_begin);
 *  - len_dev != NULL (device int32): the cache holds *len_dev rows plus this
 *    step's q_len rows, read on the device (graph-replayed verify steps);
 *    kv_len is then the largest such total the launch serves, and *len_dev
 *    must cover the visual keys (keys at or past it are not scored).
 * --------------------------------------------------------------------- */
int std_verify_attn_collect_ex(const void* q, void* k_cache, void* v_cache,
                               const void* new_k, const void* new_v, void* out,
                               int n_q, int n_kv, int q_len, int kv_len, const int32_t* len_dev, int d,
                               long long k_head_stride, long long v_head_stride,
                               long long new_head_stride, long long new_row_stride,
                               float scale, int dtype, int vis_begin, int vis_end,
                               const uint32_t* vis_mask, const int32_t* vis_rank, int n_visual,
                               float* scores, long long scores_head_stride,
                               void* workspace, size_t workspace_bytes, int32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Streaming-read ceiling (measurement helper; no counterpart in the
 * reference, which records no kernel measurement). Reads `bytes` of device
 * memory at src once and writes at most one word per workgroup to sink
 * (n_workgroups words; in practice never). bytes: a multiple of 32 KiB.
 *   mode 0/1: 256-thread workgroups issuing eight 16-byte vector loads per
 *             thread per 32 KiB tile;
 *   mode 2/3: the verify kernel's LDS DMA ring (eight waves, two tiles in
 *             flight), each tile 16 KiB from either half of the buffer;
 *   mode 4/5: the decode key split's ring (four waves, three in flight);
 *   mode 6/7: modes 3 and 5 with non-temporal loads (the policy the attention
 *             kernels use for key ranges of 4096 keys and more).
 * Modes 0, 2 and 4 give each workgroup one contiguous chunk (the tile count
 * must divide by n_workgroups); modes 1, 3, 5, 6 and 7 deal tiles round-robin.
 * ------------------------------------------------------------------------ */
int std_stream_read(const void* src, size_t bytes, int mode, int n_workgroups, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STD_HIP_H */
