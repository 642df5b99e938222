// A1: per-row fp8-e4m3fn quantisation with an fp32 (optionally UE8M0) scale.
//
// Semantics follow the reference device kernel
// operators/deepseek_v32/indexer/quantization.py:34-60: NaN-propagating row
// amax, clamp_min(1e-4), scale = amax * fl32(1/448), UE8M0 = round the scale
// bits up to a power of two, y = clamp(x / scale, +-448) cast with RNE.
// NaN follows the reference GPU's canonical NaN (scale 0x7FFFFFFF, code 0x7F).
//
// Layout: rows of `dim` elements with a row stride; the D=128 bf16 path is
// the model's shape (index K [tokens,128], index Q [tokens*64,128]) and uses
// 16 lanes per row, 8 bf16 (one 16-byte load) per lane. Other shapes and
// dtypes use one wave per row.
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

template <int kWidth>
__device__ __forceinline__ uint32_t max_abs_bits_reduce(uint32_t v) {
  // |x| as fp32 bits orders like the magnitude; any NaN (bits > 0x7F800000)
  // wins, which is the NaN-propagating max the reference uses.
#pragma unroll
  for (int offset = kWidth / 2; offset > 0; offset >>= 1) {
    uint32_t o = __shfl_xor(v, offset, kWidth);
    v = v > o ? v : o;
  }
  return v;
}

__device__ __forceinline__ float scale_from_amax_bits(uint32_t amax_bits, bool ue8m0) {
  uint32_t bits;
  if (amax_bits > 0x7F800000u) {
    bits = kCanonicalNan;
  } else {
    float amax = fmaxf(__uint_as_float(amax_bits), 1e-4f);
    bits = __float_as_uint(amax * kReciprocal448);
    if (ue8m0) bits = (bits + 0x7FFFFFu) & 0x7F800000u;
  }
  return __uint_as_float(bits);
}

__device__ __forceinline__ uint32_t quantize_one(float v, float scale, float inverse, bool ue8m0) {
  float y = ue8m0 ? v * inverse : __fdiv_rn(v, scale);
  if (y != y) return 0x7Fu;
  y = fminf(fmaxf(y, -448.0f), 448.0f);
  return f32_to_e4m3fn(y);
}

// One lane's share of a quantised row: its 8 codes and the row's folded
// weight (zeros for a row past the end).
struct QuantLane {
  uint32_t lo, hi;
  float fold;
};

// 16 lanes per 128-wide bf16 row; each lane owns 8 consecutive values. Block
// `block` of 256 threads covers rows 16 block .. 16 block + 15.
__device__ __forceinline__ QuantLane quantize_rows_d128(int64_t block, const uint16_t* __restrict__ x,
                                                   int64_t rows, int64_t row_stride,
                                                   uint8_t* __restrict__ y,
                                                   float* __restrict__ scales, int ue8m0,
                                                   const float* __restrict__ fold_in,
                                                   float* __restrict__ fold_out) {
  const int64_t row = (block * 256 + threadIdx.x) >> 4;
  const int part = threadIdx.x & 15;
  const bool live = row < rows;
  uint4 raw = make_uint4(0, 0, 0, 0);
  if (live) raw = *reinterpret_cast<const uint4*>(x + row * row_stride + part * 8);
  uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(words[i] & 0xFFFFu);
    v[2 * i + 1] = bf16_to_f32(words[i] >> 16);
  }
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t a = __float_as_uint(v[i]) & 0x7FFFFFFFu;
    m = m > a ? m : a;
  }
  m = max_abs_bits_reduce<16>(m);
  if (!live) return QuantLane{0, 0, 0.0f};
  const float scale = scale_from_amax_bits(m, ue8m0 != 0);
  const float inverse = 1.0f / scale;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= quantize_one(v[i], scale, inverse, ue8m0 != 0) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= quantize_one(v[4 + i], scale, inverse, ue8m0 != 0) << (8 * i);
  *reinterpret_cast<uint2*>(y + row * 128 + part * 8) = make_uint2(lo, hi);
  const float fold = fold_out ? fold_in[row] * scale : 0.0f;
  if (part == 0) {
    scales[row] = scale;
    if (fold_out) fold_out[row] = fold;
  }
  return QuantLane{lo, hi, fold};
}

// Partial folded query of one block of 16 index-Q rows (heads 16 g .. 16 g + 15
// of one query, g = block % 4): part[d] = sum_h w_folded[h] * q[h, d] over the
// block's heads in increasing order, one fmaf chain per dim from 0, written to
// q_fold[block, d] ([queries][4][128]). The logits kernel forms the same
// chains itself when it is not given them, so both give the same bits.
__device__ __forceinline__ void fold_partial(int64_t block, const QuantLane& mine,
                                             float* __restrict__ q_fold) {
  __shared__ uint32_t codes[16][32];
  __shared__ float fold[16];
  const int row = threadIdx.x >> 4;
  const int part = threadIdx.x & 15;
  codes[row][2 * part] = mine.lo;
  codes[row][2 * part + 1] = mine.hi;
  if (part == 0) fold[row] = mine.fold;
  __syncthreads();
  if (threadIdx.x < 128) {
    const int d = threadIdx.x;
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 16; ++h) {
      const float x = __builtin_amdgcn_cvt_f32_fp8((int)(codes[h][d >> 2] >> (8 * (d & 3))), 0);
      acc = fmaf(fold[h], x, acc);
    }
    q_fold[block * 128 + d] = acc;
  }
}

__global__ __launch_bounds__(256) void quantize_bf16_d128(const uint16_t* __restrict__ x,
                                                          int64_t rows, int64_t row_stride,
                                                          uint8_t* __restrict__ y,
                                                          float* __restrict__ scales, int ue8m0,
                                                          const float* __restrict__ fold_in,
                                                          float* __restrict__ fold_out) {
  quantize_rows_d128(blockIdx.x, x, rows, row_stride, y, scales, ue8m0, fold_in, fold_out);
}

template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p);
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p) {
  return bf16_to_f32(*p);
}
template <>
__device__ __forceinline__ float load_as_f32<_Float16>(const _Float16* p) {
  return (float)*p;
}
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p) {
  return *p;
}

// One wave per row, any width and dtype (bf16 bits, fp16, fp32).
template <typename T>
__global__ __launch_bounds__(256) void quantize_generic(const T* __restrict__ x, int64_t rows,
                                                        int64_t dim, int64_t row_stride,
                                                        uint8_t* __restrict__ y,
                                                        float* __restrict__ scales, int ue8m0,
                                                        const float* __restrict__ fold_in,
                                                        float* __restrict__ fold_out) {
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* src = x + row * row_stride;
  uint32_t m = 0;
  for (int64_t i = lane; i < dim; i += 64) {
    uint32_t a = __float_as_uint(load_as_f32<T>(src + i)) & 0x7FFFFFFFu;
    m = m > a ? m : a;
  }
  m = max_abs_bits_reduce<64>(m);
  const float scale = scale_from_amax_bits(m, ue8m0 != 0);
  const float inverse = 1.0f / scale;
  for (int64_t i = lane; i < dim; i += 64)
    y[row * dim + i] = (uint8_t)quantize_one(load_as_f32<T>(src + i), scale, inverse, ue8m0 != 0);
  if (lane == 0) {
    scales[row] = scale;
    if (fold_out) fold_out[row] = fold_in[row] * scale;
  }
}

int quantize_rows(const void* x, int dtype, int64_t rows, int64_t dim, int64_t row_stride,
                  void* out_codes, float* out_scales, int ue8m0, const float* fold_in,
                  float* fold_out, hipStream_t stream) {
  DSA_CHECK_ARG(rows >= 0 && dim >= 1 && row_stride >= dim, "invalid quantize shape");
  DSA_CHECK_ARG(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_F16 || dtype == DSA_DTYPE_F32,
                "quantize supports bf16, fp16 and fp32 inputs");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(x && out_codes && out_scales, "null pointer");
  uint8_t* y = static_cast<uint8_t*>(out_codes);
  const bool vector_path = dtype == DSA_DTYPE_BF16 && dim == 128 && row_stride % 8 == 0 &&
                           (reinterpret_cast<uintptr_t>(x) % 16) == 0;
  if (vector_path) {
    const int64_t threads = rows * 16;
    const int64_t blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(quantize_bf16_d128, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), rows, row_stride, y, out_scales, ue8m0,
                       fold_in, fold_out);
  } else {
    const int64_t blocks = (rows + 3) / 4;
    if (dtype == DSA_DTYPE_BF16)
      hipLaunchKernelGGL(quantize_generic<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const uint16_t*>(x), rows, dim, row_stride, y, out_scales,
                         ue8m0, fold_in, fold_out);
    else if (dtype == DSA_DTYPE_F16)
      hipLaunchKernelGGL(quantize_generic<_Float16>, dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const _Float16*>(x), rows, dim, row_stride, y, out_scales,
                         ue8m0, fold_in, fold_out);
    else
      hipLaunchKernelGGL(quantize_generic<float>, dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const float*>(x), rows, dim, row_stride, y, out_scales, ue8m0,
                         fold_in, fold_out);
  }
  DSA_CHECK_LAUNCH("quantize");
  return kOk;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_quantize_fp8_rows(const void* x, int dtype, int64_t rows, int64_t dim,
                                     int64_t row_stride, void* out_codes, float* out_scales,
                                     int ue8m0, hipStream_t stream) {
  return dsa::quantize_rows(x, dtype, rows, dim, row_stride, out_codes, out_scales, ue8m0, nullptr,
                            nullptr, stream);
}

extern "C" int dsa_quantize_fp8_rows_fold(const void* x, int dtype, int64_t rows, int64_t dim,
                                          int64_t row_stride, void* out_codes, float* out_scales,
                                          int ue8m0, const float* weights, float* weights_out,
                                          hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(rows <= 0 || (weights && weights_out), "null weights");
  return quantize_rows(x, dtype, rows, dim, row_stride, out_codes, out_scales, ue8m0, weights,
                       weights_out, stream);
}

namespace dsa {
namespace {

// A8 producer: pack bf16 latent+RoPE tokens (576 values) into the 656-byte
// fp8 paged record. One wave per token: lane l quantises 8 values of latent
// tile l/16 (the A1 rule, UE8M0 scale per 128-value tile); lanes 0-7 copy the
// 64 RoPE bf16 values.
// Tokens 4 block .. 4 block + 3, one wave each.
__device__ __forceinline__ void pack_tokens(int64_t block, const uint16_t* __restrict__ kv,
                                            int64_t tokens, int64_t token_offset,
                                            const int32_t* __restrict__ page_table,
                                            int64_t pages, uint8_t* __restrict__ cache,
                                            int32_t* __restrict__ status) {
  const int64_t token = block * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (token >= tokens) return;
  const int64_t logical = token_offset + token;
  const int64_t page = page_table[logical / 64];
  if (page < 0 || page >= pages) {
    if (lane == 0 && status) atomicOr(status, 1);
    return;
  }
  uint8_t* rec = cache + (page * 64 + logical % 64) * 656;
  const uint16_t* src = kv + token * 576;
  const int tile = lane >> 4;
  const int part = lane & 15;
  const uint4 raw = *reinterpret_cast<const uint4*>(src + tile * 128 + part * 8);
  const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(words[i] & 0xFFFFu);
    v[2 * i + 1] = bf16_to_f32(words[i] >> 16);
  }
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t a = __float_as_uint(v[i]) & 0x7FFFFFFFu;
    m = m > a ? m : a;
  }
  m = max_abs_bits_reduce<16>(m);
  const float scale = scale_from_amax_bits(m, true);
  const float inverse = 1.0f / scale;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= quantize_one(v[i], scale, inverse, true) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= quantize_one(v[4 + i], scale, inverse, true) << (8 * i);
  *reinterpret_cast<uint2*>(rec + tile * 128 + part * 8) = make_uint2(lo, hi);
  if (part == 0) *reinterpret_cast<float*>(rec + 512 + 4 * tile) = scale;
  if (lane < 8)
    *reinterpret_cast<uint4*>(rec + 528 + lane * 16) =
        *reinterpret_cast<const uint4*>(src + 512 + lane * 8);
}

__global__ __launch_bounds__(256) void kv_pack_fp8(const uint16_t* __restrict__ kv,
                                                   int64_t tokens, int64_t token_offset,
                                                   const int32_t* __restrict__ page_table,
                                                   int64_t pages, uint8_t* __restrict__ cache,
                                                   int32_t* __restrict__ status) {
  pack_tokens(blockIdx.x, kv, tokens, token_offset, page_table, pages, cache, status);
}

// The three small stages of a layer step in one launch: blocks [0, nq) quantise
// the indexer Q rows and fold their scales into the head weights, blocks
// [nq, nq + nk) quantise the new index-K rows into the resident cache, and the
// rest pack the new KV tokens into the fp8 paged cache. All three are
// independent of each other.
__global__ __launch_bounds__(256) void layer_prologue(
    const uint16_t* __restrict__ q, int64_t q_rows, const float* __restrict__ weights,
    uint8_t* __restrict__ q_codes, float* __restrict__ q_scales, float* __restrict__ w_folded,
    float* __restrict__ q_fold, const uint16_t* __restrict__ k, int64_t k_rows,
    uint8_t* __restrict__ k_codes,
    float* __restrict__ k_scales, const uint16_t* __restrict__ kv, int64_t tokens,
    int64_t token_offset, const int32_t* __restrict__ page_table, int64_t pages,
    uint8_t* __restrict__ cache, int32_t* __restrict__ status, int64_t nq, int64_t nk) {
  const int64_t b = blockIdx.x;
  if (b < nq) {
    const QuantLane mine = quantize_rows_d128(b, q, q_rows, 128, q_codes, q_scales, 1, weights, w_folded);
    if (q_fold) fold_partial(b, mine, q_fold);
  } else if (b < nq + nk) {
    quantize_rows_d128(b - nq, k, k_rows, 128, k_codes, k_scales, 1, nullptr, nullptr);
  } else {
    pack_tokens(b - nq - nk, kv, tokens, token_offset, page_table, pages, cache, status);
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_kv_pack_fp8(const void* kv, int64_t tokens, int64_t token_offset,
                               const int32_t* page_table, int64_t pages, void* cache,
                               int32_t* status, hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(tokens >= 0 && token_offset >= 0 && pages >= 0, "invalid pack shape");
  DSA_CHECK_ARG(token_offset + tokens <= pages * 64, "tokens exceed the paged cache");
  if (tokens == 0) return kOk;
  DSA_CHECK_ARG(kv && page_table && cache, "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(kv) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(cache) % 16 == 0,
                "kv and cache must be 16-byte aligned");
  hipLaunchKernelGGL(kv_pack_fp8, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(kv), tokens, token_offset, page_table, pages,
                     static_cast<uint8_t*>(cache), status);
  DSA_CHECK_LAUNCH("fp8 KV pack");
  return kOk;
}

extern "C" int dsa_layer_prologue_fp8(const void* q, int64_t q_rows, const float* weights,
                                      void* q_codes, float* q_scales, float* w_folded,
                                      float* q_fold, const void* k, int64_t k_rows, void* k_codes,
                                      float* k_scales, const void* kv, int64_t tokens,
                                      int64_t token_offset, const int32_t* page_table,
                                      int64_t pages, void* cache, int32_t* status,
                                      hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(q_rows >= 0 && k_rows >= 0 && tokens >= 0 && token_offset >= 0 && pages >= 0,
                "invalid prologue shape");
  DSA_CHECK_ARG(token_offset + tokens <= pages * 64, "tokens exceed the paged cache");
  DSA_CHECK_ARG((q_rows == 0 || (q && weights && q_codes && q_scales && w_folded)) &&
                    (k_rows == 0 || (k && k_codes && k_scales)) &&
                    (tokens == 0 || (kv && page_table && cache)),
                "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(kv) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(cache) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(q_codes) % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(k_codes) % 8 == 0,
                "prologue inputs must be 16-byte and code outputs 8-byte aligned");
  DSA_CHECK_ARG(q_fold == nullptr || q_rows % 64 == 0,
                "the folded query needs whole queries of 64 index-Q rows");
  const int64_t nq = (q_rows * 16 + 255) / 256;
  const int64_t nk = (k_rows * 16 + 255) / 256;
  const int64_t nt = (tokens + 3) / 4;
  if (nq + nk + nt == 0) return kOk;
  DSA_CHECK_ARG(nq + nk + nt < 0x7FFFFFFF, "prologue too large for one launch");
  hipLaunchKernelGGL(layer_prologue, dim3((unsigned)(nq + nk + nt)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(q), q_rows, weights,
                     static_cast<uint8_t*>(q_codes), q_scales, w_folded, q_rows ? q_fold : nullptr,
                     static_cast<const uint16_t*>(k), k_rows, static_cast<uint8_t*>(k_codes),
                     k_scales, static_cast<const uint16_t*>(kv), tokens, token_offset, page_table,
                     pages, static_cast<uint8_t*>(cache), status, nq, nk);
  DSA_CHECK_LAUNCH("layer prologue");
  return kOk;
}
