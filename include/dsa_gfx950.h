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
 * A7 - sparse MLA over flat bf16 records. Replaces sparse_mla /
 * sparse_mla_from_pool (FlashMLA flash_mla_sparse_fwd),
 * operators/deepseek_v32/attention/device_only/mla.py:156-181 and
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

#ifdef __cplusplus
}
#endif

#endif /* DSA_GFX950_H_ */
