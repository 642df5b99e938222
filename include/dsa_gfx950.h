/*
 * dsa_gfx950.h - C ABI of libdsa_gfx950.so, the MI355X (gfx950) kernels of
 * the DeepSeek-V3.2 sparse-attention (DSA) prefill path.
 *
 * Conventions for every entry point:
 *   - return 0 on success; nonzero on failure, with a message available from
 *     dsa_last_error() on the calling host thread;
 *   - all tensor arguments are raw device pointers (or pinned host pointers
 *     where stated), sizes and strides are int64 element counts;
 *   - work is enqueued on `stream` and never synchronised; outputs are valid
 *     once the stream reaches that point;
 *   - no entry point allocates device memory; scratch comes from the caller.
 *
 * Reference interfaces each entry replaces are cited as path:line relative to
 * the chiakicage/cxldsagr checkout.
 */
#ifndef DSA_GFX950_H_
#define DSA_GFX950_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_ABI_VERSION 1

/* Element types accepted by dsa_quantize_fp8_rows. */
#define DSA_DTYPE_BF16 0
#define DSA_DTYPE_F16 1
#define DSA_DTYPE_F32 2

/* Element types of the optional device valid_count of dsa_gather_records. */
#define DSA_COUNT_I64 0
#define DSA_COUNT_U32 1

/* Copy the last error message of this host thread into `buffer` (always
 * NUL-terminated when size > 0). Returns the message length. */
int dsa_last_error(char* buffer, size_t size);

/* ABI version of the loaded library (DSA_ABI_VERSION). */
int dsa_abi_version(void);

/*
 * A1 - indexer fp8 quantisation.
 * Replaces quantize_index / its Triton kernel,
 * operators/deepseek_v32/indexer/quantization.py:63-88 (kernel :34-60).
 * x: `rows` rows of `dim` elements of `dtype`, row stride `row_stride`.
 * out_codes: uint8 e4m3fn [rows, dim] contiguous; out_scales: f32 [rows].
 * ue8m0 != 0 rounds each scale up to a power of two.
 */
int dsa_quantize_fp8_rows(const void* x, int dtype, int64_t rows, int64_t dim,
                          int64_t row_stride, void* out_codes, float* out_scales, int ue8m0,
                          hipStream_t stream);

/*
 * A1 + A2 - the same quantisation with the q-scale folded into the indexer
 * head weights in the same pass: weights_out[i] = weights[i] * out_scales[i]
 * (fp32 multiply) for every row i. Rows are (query, head) pairs in order, so
 * weights / weights_out are the contiguous f32 [queries, heads] matrices.
 * Replaces quantize_index (quantization.py:63-88) followed by the weight fold
 * `weights * q_scale[..., 0]` of models/deepseek_v32/projections.py:241-244.
 */
int dsa_quantize_fp8_rows_fold(const void* x, int dtype, int64_t rows, int64_t dim,
                               int64_t row_stride, void* out_codes, float* out_scales, int ue8m0,
                               const float* weights, float* weights_out, hipStream_t stream);

/*
 * A4 - fp8 MQA indexer logits with the causal -inf tail.
 * Replaces the resident branch of logits(),
 * operators/deepseek_v32/indexer/echo.py:299-410 (DeepGEMM
 * fp8_fp4_mqa_logits at :386-393 plus the tail mask at :397-409).
 * q: e4m3 [rows, 64, 128]; k: e4m3 [columns, 128]; weights: f32 [rows, 64];
 * kscale: f32 [columns]; starts/ends: int32 [rows] or both NULL (then
 * [0, query_start + i + 1)); out: f32 [rows, ldo] with ldo >= columns, every
 * column outside [starts[i], ends[i]) and every padded column is -inf.
 */
int dsa_indexer_logits_fp8(const void* q, const void* k, const float* weights,
                           const float* kscale, const int32_t* starts, const int32_t* ends,
                           int64_t query_start, int64_t rows, int64_t columns, int64_t ldo,
                           float* out, hipStream_t stream);

/*
 * A4, the same contract and the same bits as dsa_indexer_logits_fp8, given
 * q_fold: f32 [rows, 4, 128], the partial folded queries that
 * dsa_layer_prologue_fp8 writes (16-byte aligned). The kernel then skips
 * forming them itself. Same reference interface as dsa_indexer_logits_fp8
 * (echo.py:299-410); the layer step calls this one.
 */
int dsa_indexer_logits_fp8_folded(const void* q, const void* k, const float* weights,
                                  const float* kscale, const int32_t* starts, const int32_t* ends,
                                  int64_t query_start, int64_t rows, int64_t columns,
                                  int64_t ldo, const float* q_fold, float* out,
                                  hipStream_t stream);

/*
 * A6 - exact top-k, k <= 2048, sorted descending, SMALL ties, -1 ids for
 * non-finite values. Replaces exact_topk,
 * operators/deepseek_v32/indexer/selection.py:62-113 (FlashInfer radix_topk
 * at :14-34 and the mask kernel at :37-59).
 * scores: f32 [rows, ld] (first `columns` used); values f32 / indices int32
 * [rows, out_ld], first min(k, columns) entries of each row written.
 */
int dsa_topk_radix(const float* scores, int64_t rows, int64_t columns, int64_t ld, int64_t k,
                   float* values, int32_t* indices, int64_t out_ld, hipStream_t stream);

/*
 * A6, same contract and results as dsa_topk_radix, with each row of 8192 or
 * more columns split over two work-groups (each selects and sorts the top
 * min(k, half) keys of its half into the workspace; a second launch on the
 * same stream merges the two lists of every row), so that a launch of Q rows
 * occupies 2Q compute units. Replaces the same exact_topk
 * (selection.py:62-113). workspace: device memory of the size
 * dsa_topk_workspace_bytes(rows, &bytes) stores, 8-byte aligned, no
 * initialisation needed; calls that overlap on different streams need
 * distinct workspaces. Shorter rows run the one-work-group kernel.
 */
int dsa_topk_workspace_bytes(int64_t rows, int64_t* bytes);
int dsa_topk_radix_split(const float* scores, int64_t rows, int64_t columns, int64_t ld, int64_t k,
                         float* values, int32_t* indices, int64_t out_ld, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream);

/*
 * A6, dsa_topk_radix_split without a workspace argument and without any
 * allocation: the half-row lists go to a library-owned device array of
 * 512 rows x 2 x 2048 x 8 bytes (16 MiB per GPU, held until the process
 * ends), addressed through hipGetSymbolAddress once per device. At most 512
 * rows per call; more is rejected. Same results as dsa_topk_radix_split.
 * Calls that overlap on one GPU (several streams) race on the array; the
 * contents of one call are never read by the next. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
int dsa_topk_radix_split_static(const float* scores, int64_t rows, int64_t columns, int64_t ld,
                                int64_t k, float* values, int32_t* indices, int64_t out_ld,
                                hipStream_t stream);

/*
 * A4, dsa_indexer_logits_fp8 (q_fold NULL) or dsa_indexer_logits_fp8_folded
 * (q_fold given) with the same output bits, that also adds to digit_counts
 * (uint32 [rows, 2048], 4-byte aligned) the number of each row's scores in
 * columns [0, columns) by the top 11 bits of their fp32 radix key (the
 * counts dsa_topk_radix_digits takes; masked and -inf columns included).
 * The counts are added, so they start from zero for a fresh histogram.
 * Replaces the same logits() (echo.py:299-410) with the per-query coarse
 * score buckets of the reference's ECHO kernel
 * (indexer/csrc/echo_logits.cuh:497-561) at the top-k's digit width.
 */
int dsa_indexer_logits_fp8_counted(const void* q, const void* k, const float* weights,
                                   const float* kscale, const int32_t* starts,
                                   const int32_t* ends, int64_t query_start, int64_t rows,
                                   int64_t columns, int64_t ldo, const float* q_fold, float* out,
                                   uint32_t* digit_counts, hipStream_t stream);

/*
 * A6 given the level-0 radix histogram: same contract and results as
 * dsa_topk_radix. The workspace (dsa_indexer_topk_workspace_bytes(rows,
 * columns, &bytes), 8-byte aligned, all zero before the first use) starts with
 * uint32 [rows, 2048] digit counts, which the caller adds for each row before
 * the call: the number of the row's scores in columns [0, columns) whose
 * fp32 radix key (bits | 0x80000000 for non-negative values, ~bits for
 * negative ones) has each value of its top 11 bits, as
 * dsa_indexer_logits_fp8_counted accumulates them. A first launch reads each
 * row once over several work-groups and lists only its keys at or above the
 * digit where the count-th largest key lies; a second launch, one
 * work-group per row, splits that digit's keys, sorts and writes the row.
 * The call leaves the counts and the list fill all zero again. The layout
 * depends on `rows`: before a call with another row count than the last one,
 * zero the workspace again (a workspace that is not all zero where the
 * layout needs it costs the selection from the counts - those rows are
 * selected from their scores - never the results or memory outside it).
 * A row whose counts do not sum to `columns` runs the full selection over its
 * scores (same results). Replaces the same exact_topk (selection.py:62-113);
 * the counts follow the per-query coarse score buckets of the reference's
 * ECHO kernel (indexer/csrc/echo_logits.cuh:497-561). Calls that overlap on
 * different streams need distinct workspaces.
 */
int dsa_indexer_topk_workspace_bytes(int64_t rows, int64_t columns, int64_t* bytes);
int dsa_topk_radix_digits(const float* scores, int64_t rows, int64_t columns, int64_t ld, int64_t k,
                          float* values, int32_t* indices, int64_t out_ld, void* workspace,
                          int64_t workspace_bytes, hipStream_t stream);

/*
 * A4 + A6 fused: dsa_indexer_logits_fp8_counted into scores [rows, ldo]
 * with the start of the workspace as its digit counts, then
 * dsa_topk_radix_digits over scores[:, 0:columns) with that workspace: the
 * same scores, values and indices as the two calls logits then
 * dsa_topk_radix. Workspace as for dsa_topk_radix_digits (all zero before
 * the first use with a given row count; the counts and fill are zero again
 * after every call).
 * Calls that overlap on different streams need distinct workspaces. Replaces the
 * reference's logits() followed by exact_topk() in the indexer step
 * (models/deepseek_v32/attention.py:338-363, echo.py:299-410,
 * selection.py:62-113).
 */
int dsa_indexer_topk_fp8(const void* q, const void* k, const float* weights, const float* kscale,
                         const int32_t* starts, const int32_t* ends, int64_t query_start,
                         int64_t rows, int64_t columns, int64_t ldo, const float* q_fold,
                         float* scores, int64_t topk, float* values, int32_t* indices,
                         int64_t out_ld, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream);

/*
 * A4 + A6 fused without the score matrix (the fused indexer step that
 * writes only top-k candidates): the same values and indices as
 * dsa_indexer_logits_fp8 followed by dsa_topk_radix over its [rows, columns]
 * scores, bit for bit, for every input. Replaces the reference's logits()
 * followed by exact_topk() in the indexer step
 * (models/deepseek_v32/attention.py:338-363, echo.py:299-410,
 * selection.py:62-113); the reference's ECHO kernel likewise buckets each
 * query's scores against a per-query offset estimated ahead of the call
 * (indexer/csrc/echo_logits.cuh:497-561, indexer/prefetch_hint.py:38-85).
 *
 * Three launches, also available one by one:
 *  - dsa_indexer_floors_fp8: per row a floor (an fp32 radix key) estimated
 *    from the row's scores at about 1/64 of its visible columns, so that the
 *    row almost surely holds at least min(topk, columns) scores at or above
 *    it; 0 for rows of fewer than 8192 visible columns; written to
 *    floors[2 row] and floors[2 row + 1] (uint32 [rows][2]);
 *  - dsa_indexer_logits_fp8_emit: the logits kernel writes, per row and key
 *    split, only the composite keys (radix(v) << 32 | ~column) of the scores
 *    at or above the row's floor into the workspace lists; a split whose list
 *    fills up stores the rest of its scores into `scores` instead, and rows
 *    with floor 0 are stored there in full;
 *  - dsa_indexer_emit_topk: per row, the exact top-k of the candidates when
 *    there are at least min(topk, columns) of them (they then hold the row's
 *    top); otherwise the row's scores are recomputed into `scores` with the
 *    logits kernel's arithmetic and selected from (exact, slow, rare).
 * `scores` is f32 [rows, ldo] with ldo = columns rounded up to 256: scratch
 * that holds only stored rows and spilled columns afterwards. q_fold as for
 * dsa_indexer_logits_fp8_folded (may be NULL). list_cap = 0 picks the list
 * length per (row, split) (an eighth of the split); a smaller one makes
 * splits spill earlier (for tests). The workspace (256-byte aligned, size
 * from dsa_indexer_select_workspace_bytes with the same rows, columns and
 * list_cap on the same device) holds floors u32 [rows][2] (a row's floor is
 * the smaller of its two entries; dsa_indexer_floors_fp8 writes one
 * estimate twice), records and lists;
 * it needs no initialisation, and calls that overlap on different streams
 * need distinct workspaces and score buffers. A caller may overwrite the
 * floors between the first two launches (a floor too high for a row only
 * sends that row to the recompute).
 */
int dsa_indexer_select_workspace_bytes(int64_t rows, int64_t columns, int64_t list_cap,
                                       int64_t* bytes);
int dsa_indexer_floors_fp8(const void* q, const void* k, const float* weights, const float* kscale,
                           const int32_t* starts, const int32_t* ends, int64_t query_start,
                           int64_t rows, int64_t columns, int64_t topk, uint32_t* floors,
                           hipStream_t stream);
int dsa_indexer_logits_fp8_emit(const void* q, const void* k, const float* weights,
                                const float* kscale, const int32_t* starts, const int32_t* ends,
                                int64_t query_start, int64_t rows, int64_t columns, int64_t ldo,
                                const float* q_fold, float* scores, int64_t list_cap,
                                void* workspace, int64_t workspace_bytes, hipStream_t stream);
int dsa_indexer_emit_topk(const void* q, const void* k, const float* weights, const float* kscale,
                          const int32_t* starts, const int32_t* ends, int64_t query_start,
                          int64_t rows, int64_t columns, const float* q_fold, float* scores,
                          int64_t topk, float* values, int32_t* indices, int64_t out_ld,
                          int64_t list_cap, const void* workspace, int64_t workspace_bytes,
                          hipStream_t stream);
/* The three launches above in order, with list_cap = 0 (floors at the start
 * of the workspace). */
int dsa_indexer_select_fp8(const void* q, const void* k, const float* weights, const float* kscale,
                           const int32_t* starts, const int32_t* ends, int64_t query_start,
                           int64_t rows, int64_t columns, const float* q_fold, float* scores,
                           int64_t topk, float* values, int32_t* indices, int64_t out_ld,
                           void* workspace, int64_t workspace_bytes, hipStream_t stream);


/*
 * A8 producer - pack bf16 [tokens, 576] (512 latent + 64 RoPE) into the
 * 656-byte fp8 paged record: 4 e4m3 tiles of 128 (A1 rule, UE8M0), 4 fp32
 * tile scales, 64 raw bf16 RoPE values. Token i goes to logical position
 * token_offset + i, physical row page_table[pos / 64] * 64 + pos % 64 of
 * cache uint8 [pages * 64, 656]. A page number outside [0, pages) skips the
 * token and ORs 1 into *status (may be NULL). No reference counterpart: the
 * reference appends bf16 records (models/deepseek_v32/attention.py:400-401).
 */
int dsa_kv_pack_fp8(const void* kv, int64_t tokens, int64_t token_offset,
                    const int32_t* page_table, int64_t pages, void* cache, int32_t* status,
                    hipStream_t stream);

/*
 * Layer-step prologue in one launch: the fold variant of the A1 quantiser on
 * q_rows contiguous bf16 [q_rows, 128] indexer-Q rows (UE8M0; q_codes e4m3
 * [q_rows, 128], q_scales f32 [q_rows], w_folded = weights * q_scales), the
 * A3 quantiser on k_rows bf16 [k_rows, 128] new index-K rows into k_codes /
 * k_scales, and dsa_kv_pack_fp8 of `tokens` new bf16 [tokens, 576] KV
 * records. No reference counterpart as one entry: it replaces the three
 * launches of models/deepseek_v32/projections.py:241-244 +
 * quantization.py:63-88, attention.py:323-326 and attention.py:400-401 in a
 * layer step. Results equal those three entry points bit for bit. q_fold
 * (optional, f32 [q_rows / 64, 4, 128]; q_rows a multiple of 64) receives
 * the partial folded queries for dsa_indexer_logits_fp8_folded: entry
 * [i, g, d] = sum over heads h = 16g .. 16g + 15 of w_folded[i, h] *
 * q_codes[i, h, d], one fmaf chain per entry in increasing h.
 */
int dsa_layer_prologue_fp8(const void* q, int64_t q_rows, const float* weights, void* q_codes,
                           float* q_scales, float* w_folded, float* q_fold, const void* k,
                           int64_t k_rows, void* k_codes, float* k_scales, const void* kv,
                           int64_t tokens, int64_t token_offset, const int32_t* page_table,
                           int64_t pages, void* cache, int32_t* status, hipStream_t stream);

/*
 * dsa_layer_prologue_fp8 that also writes the per-row floors of the
 * candidate top-k into `floors` (uint32 [q_rows / 64][2]: two estimates per
 * row from the two halves of its sample, the row's floor being the smaller),
 * for a layer step whose queries are the causal rows
 * history .. history + q_rows / 64 - 1 over the resident index keys
 * key_cache e4m3 [history + ..., 128] / key_cache_scales f32: each row's
 * floor is sampled from columns [0, history) (the new keys are written by
 * the same launch). Pass the select workspace's floors (its first bytes) and
 * then call dsa_indexer_logits_fp8_emit and dsa_indexer_emit_topk. No
 * reference counterpart (the reference has no floors); the same quantised
 * outputs as dsa_layer_prologue_fp8.
 */
int dsa_layer_prologue_floors_fp8(const void* q, int64_t q_rows, const float* weights,
                                  void* q_codes, float* q_scales, float* w_folded, float* q_fold,
                                  const void* k, int64_t k_rows, void* k_codes, float* k_scales,
                                  const void* kv, int64_t tokens, int64_t token_offset,
                                  const int32_t* page_table, int64_t pages, void* cache,
                                  int32_t* status, const void* key_cache,
                                  const float* key_cache_scales, int64_t history, int64_t topk,
                                  uint32_t* floors, hipStream_t stream);

/*
 * Indexer input producers: the indexer half of the projection step after
 * its GEMMs, in one launch. Replaces, in the reference's project()
 * (models/deepseek_v32/projections.py:182-257), the K LayerNorm of
 * _project_index_k (:114-121), apply_rope_pair(index_q, index_k, angles,
 * interleaved=False) (:236-238; rotary.py:47-56,69-85), the two
 * quantize_index calls (:239-240) and the weight scaling (:241-242), and
 * the runner's index-cache write (models/deepseek_v32/attention.py:323-326).
 *
 * q_proj: bf16 [tokens, 64, 128] (index_wq output); k_proj: bf16
 * [tokens, 128] (index_wk output); head_logits: f32 [tokens, 64]
 * (weights_proj output); weights_out[t,h] = ((head_logits * pre) *
 * q_scale) * post (the model's pre = 64^-1/2, post = 128^-1/2).
 * K: y = LayerNorm(k_proj) with norm_weight/norm_bias f32 [128], norm_eps,
 * rounded to bf16. Q and K: RoPE on dims [0, 64), dim i with dim i + 32,
 * cos/sin from row rope_rows[t] (or t when rope_rows is NULL) of cos_sin
 * f32 [table_rows, 64] (32 cos then 32 sin), rounded to bf16; then the A1
 * quantiser with UE8M0 scales. Outputs: q_codes e4m3 [tokens, 64, 128],
 * q_scales f32 [tokens, 64], weights_out f32 [tokens, 64], optional q_fold
 * f32 [tokens, 4, 128] (as dsa_layer_prologue_fp8), k_codes e4m3
 * [tokens, 128] and k_scales f32 [tokens] (the index cache rows). With kv
 * non-NULL the new KV tokens bf16 [tokens, 576] are also packed into the fp8
 * paged cache at token_offset (as dsa_kv_pack_fp8). status (optional,
 * int32): bit 0 a page outside the cache, bit 1 a RoPE row outside the
 * table (row 0 used instead).
 */
int dsa_index_producer_fp8(const void* q_proj, int64_t tokens, const float* head_logits,
                           float head_pre_scale, float head_post_scale, const void* k_proj,
                           const float* norm_weight, const float* norm_bias, float norm_eps,
                           const float* cos_sin, int64_t table_rows, const int32_t* rope_rows,
                           void* q_codes, float* q_scales, float* weights_out, float* q_fold,
                           void* k_codes, float* k_scales, const void* kv, int64_t token_offset,
                           const int32_t* page_table, int64_t pages, void* cache,
                           int32_t* status, hipStream_t stream);

/*
 * dsa_index_producer_fp8 that also writes the per-row floors of the
 * candidate top-k into `floors` (uint32 [tokens][2], as
 * dsa_layer_prologue_floors_fp8 writes them), for a layer step whose queries
 * are the causal rows history .. history + tokens - 1 over the resident
 * index keys key_cache e4m3 [history + ..., 128] / key_cache_scales f32:
 * each row's floor is sampled from columns [0, history), scored with the
 * query's own rotated, quantised rows and head weights (the same bits the
 * launch writes to q_codes and weights_out). No reference counterpart (the
 * reference has no floors); the same producer outputs as
 * dsa_index_producer_fp8.
 */
int dsa_index_producer_floors_fp8(
    const void* q_proj, int64_t tokens, const float* head_logits, float head_pre_scale,
    float head_post_scale, const void* k_proj, const float* norm_weight, const float* norm_bias,
    float norm_eps, const float* cos_sin, int64_t table_rows, const int32_t* rope_rows,
    void* q_codes, float* q_scales, float* weights_out, float* q_fold, void* k_codes,
    float* k_scales, const void* kv, int64_t token_offset, const int32_t* page_table,
    int64_t pages, void* cache, int32_t* status, const void* key_cache,
    const float* key_cache_scales, int64_t history, int64_t topk, uint32_t* floors,
    hipStream_t stream);

/*
 * A7 - sparse MLA over flat bf16 records. Replaces sparse_mla /
 * sparse_mla_from_pool (FlashMLA flash_mla_sparse_fwd),
 * operators/deepseek_v32/attention/device_only/mla.py:90-115 and
 * operators/deepseek_v32/attention/offload/mla.py:12-20.
 * q: bf16 [rows, heads, 576] (heads a multiple of 64); kv: bf16
 * [kv_rows, 576]; indices: int32 [rows, topk], ids outside [0, kv_rows) are
 * padding; out: bf16 [rows, heads, 512]. softmax scale `scale`.
 */
int dsa_sparse_mla_bf16(const void* q, int64_t rows, int64_t heads, const void* kv,
                        int64_t kv_rows, const int32_t* indices, int64_t topk, float scale,
                        void* out, hipStream_t stream);

/*
 * A7 over the A8 fp8 paged cache (no reference counterpart; same semantics
 * as dsa_sparse_mla_bf16 on the dequantised records). cache: uint8
 * [pages * 64, 656]; page_table: int32 logical page -> physical page; ids
 * outside [0, n_tokens) (or mapped outside the cache) are padding.
 */
int dsa_sparse_mla_fp8_paged(const void* q, int64_t rows, int64_t heads, const void* cache,
                             int64_t pages, const int32_t* page_table, int64_t n_tokens,
                             const int32_t* indices, int64_t topk, float scale, void* out,
                             hipStream_t stream);

/*
 * A11 - gather whole records from pinned host memory into device memory,
 * device[device_ids[r]] = host[host_ids[r]] for r < count, or for
 * r < *valid_count when valid_count (a device int64 or uint32 scalar, kind
 * DSA_COUNT_*) is given. Replaces gather_host_records,
 * operators/common/kv_transfer.py:21-68 (kernel gather_records,
 * operators/common/csrc/kv_transfer.cu:14-64).
 * host: pinned host allocation (hipHostMalloc / torch pin_memory) of
 * host_rows x row_bytes; device: device_rows x row_bytes; ids int64 on the
 * device. max_blocks bounds the grid (0 = automatic). An id out of range
 * skips its row and ORs 1 into *status, a valid_count outside [0, count]
 * copies nothing and ORs 2 (status may be NULL): the reference traps instead.
 */
int dsa_gather_records(const void* host, int64_t host_rows, void* device, int64_t device_rows,
                       int64_t row_bytes, const int64_t* host_ids, const int64_t* device_ids,
                       int64_t count, const void* valid_count, int count_kind, int64_t max_blocks,
                       int32_t* status, hipStream_t stream);

/*
 * A11 - contiguous host-to-device record copy on `stream` (hipMemcpyAsync).
 * Replaces copy_host_records_async, operators/common/kv_transfer.py:71-103
 * (copy_contiguous, kv_transfer.cu:83-99); spans are checked by the caller.
 */
int dsa_copy_records_h2d(const void* host, void* device, int64_t bytes, hipStream_t stream);

/*
 * A10 - workspace size in bytes for dsa_pool_recall on a pool of `slots`
 * slots and sequences of at most `history_capacity` host-backed tokens.
 */
int dsa_pool_workspace_bytes(int64_t slots, int64_t history_capacity, int64_t* bytes);

/*
 * A10 - exact recall of a top-k selection into the HBM token pool, then the
 * logical -> physical map. Replaces SparseTokenCache.ensure /
 * _ensure_sparse_from_topk, cache/sparse_token_cache.py:502-569 and :616-739
 * (native stages sparse_selection_classify / allocate / gather_records /
 * publish / map, operators/deepseek_v32/indexer/cache_ops.py:303-1016).
 * indices: int32 [n] logical ids (-1 padding); page_table: int32 logical page
 * -> global host page; ids in [0, history_end) are host-backed, ids in
 * [transient_start, written) (transient_start >= 0) are candidate rows
 * slots + 1 + id - transient_start, which must lie inside record_rows (else
 * the call fails); every other id, including one at or past `written`, maps
 * to -1 (padding). Pool state: h2d int32 [host_rows] (MISSING = INT32_MAX),
 * d2h / priority int64 [slots + 1] (slot 0 is the sentinel), records
 * [record_rows, record_bytes] on the device, host records pinned
 * [host_rows, record_bytes]. Hits are stamped protect_stamp, recalled slots
 * chosen_stamp; stamps form a FIFO clock: every priority already stored is
 * below this call's chosen_stamp (victims are ordered by priority, then slot).
 * stats int64 [4] accumulates union, recalled, evicted.
 * status bits: 4 = an id at or past `written`, 8 = the union did not fit.
 * With history_end > slots the caller must pass union_checked != 0 after
 * checking the union size. physical: int32 [n]. Not for HIP graph capture:
 * the victim sort (rocPRIM) clears its buffers with hipMemsetAsync.
 */
int dsa_pool_recall(const int32_t* indices, int64_t n, const int32_t* page_table,
                    int64_t history_end, int64_t written, int64_t transient_start, int64_t slots,
                    const void* host, int64_t host_rows, void* records, int64_t record_rows,
                    int64_t record_bytes, int32_t* h2d, int64_t* d2h, int64_t* priority,
                    int64_t protect_stamp, int64_t chosen_stamp, void* workspace,
                    int64_t workspace_bytes, int64_t history_capacity, int union_checked,
                    int64_t* stats, int32_t* status, int32_t* physical, hipStream_t stream);

/*
 * A10 for overlapped multi-user recall (no counterpart in the reference, whose
 * users recall one after another): dsa_pool_recall with two more arguments.
 * keep_floor >= 0 (below protect_stamp) also keeps every occupied slot whose
 * priority is >= keep_floor out of the victims - pass the protect_stamp of the
 * previous recall while that selection is still read by sparse MLA on another
 * stream. candidate_offset >= 0 moves this call's candidate rows to
 * slots + 1 + candidate_offset + id - transient_start (alternate halves of the
 * candidate rows between users in flight). The victims then differ from the
 * sequential FIFO order; every selected id still maps to a row holding its
 * record. gather_stream (null: `stream`) takes the gather of the missing
 * records, ordered after the slot assignment on `stream`; the next recall on
 * `stream` may then run while it copies, given another workspace, and readers
 * of the records wait for gather_stream. With keep_floor = -1,
 * candidate_offset = 0 and no gather stream it is dsa_pool_recall.
 */
int dsa_pool_recall_pipelined(const int32_t* indices, int64_t n, const int32_t* page_table,
                              int64_t history_end, int64_t written, int64_t transient_start,
                              int64_t slots, const void* host, int64_t host_rows, void* records,
                              int64_t record_rows, int64_t record_bytes, int32_t* h2d,
                              int64_t* d2h, int64_t* priority, int64_t protect_stamp,
                              int64_t chosen_stamp, void* workspace, int64_t workspace_bytes,
                              int64_t history_capacity, int union_checked, int64_t* stats,
                              int32_t* status, int32_t* physical, int64_t keep_floor,
                              int64_t candidate_offset, hipStream_t stream,
                              hipStream_t gather_stream);

/*
 * A10 release of a session's host rows from one layer's pool maps
 * (cache/sparse_token_pool.py:697-710, release_ids): for every host row of
 * the session's pages (page_table int32 [pages], 64 rows per page) that is
 * resident, its slot is freed (d2h = MISSING, priority = -1) and h2d of the
 * row becomes MISSING. A page outside [0, host_rows / 64) or an h2d entry
 * outside [1, slots] ORs 1 into *status (may be NULL) and is skipped.
 */
int dsa_pool_release_rows(const int32_t* page_table, int64_t pages, int64_t host_rows,
                          int32_t* h2d, int64_t* d2h, int64_t* priority, int64_t slots,
                          int32_t* status, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_GFX950_H_ */
