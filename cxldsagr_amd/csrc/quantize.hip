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
#include "logits_core.h"
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

// Floors of the candidate top-k (logits_core.h: floor_rank, row_floor,
// floor_of_samples) for the layer step: two 256-thread blocks per query row
// i, block h scoring the interleaved half h of the row's sample columns
// (2m + h for m < n/2) of the resident history [0, history) - the new keys
// are being written by this launch - and writing its own estimate to
// floors[2i + h]; the row's floor is the smaller of the two, which is too
// high only when both are, so each half takes a 3.5 sigma margin. Each block
// quantises the row's 64 index-Q head rows (the A1 scale; the e4m3 codes by
// the hardware conversion - the floor is an estimate, and the exact codes
// are the Q blocks') and scores its samples with four MFMAs per 16 (each
// wave a quarter of them, all 64 heads; the MFMAs of one group are issued
// before the previous group's head sum). The query loads are issued first
// and the sample loads after the quantisation: issued before it, they
// delayed the query rows it waits for (~1.5k ticks per block).
// The prologue launches are bound by load latency (808 blocks at configs
// 1+2, two thirds of them short): three resident blocks per CU (168
// registers, no scratch) instead of the two that 190 registers allowed took
// the launch from 10.2 to 9.1 us (4.2 us without floor blocks) and config
// 4's from 41 to 35 us; four would spill.
constexpr int kPrologueBlocksPerCu = 3;
constexpr int kPrologueFloorSamples = 2048;  // per row (both halves)
constexpr int kPrologueFloorBatch = 8;  // 16-sample groups per wave in flight together
constexpr float kPrologueFloorSigmas = 3.5f;

struct FloorArgs {
  const uint8_t* keys;      // resident index-K codes [history + ...][128]
  const float* key_scales;  // [history + ...]
  int64_t history;          // sample columns [0, history); row i sees history + i + 1
  int count;                // min(topk, columns)
  uint32_t* floors;         // [rows][2]
};

// The floor blocks of the index producer take the index-Q row before RoPE
// (the Q projection's output) and form the head weights from the head
// logits: the query's RoPE row and the weight inputs. With `cos_sin` null the
// query rows are already rotated and `weights` holds the head weights.
struct FloorProducer {
  const float* cos_sin;  // [table_rows, 64]: cos of the 32 angles, then their sin
  const int32_t* rows;   // RoPE table row of each query, or null: query i uses row i
  int64_t table_rows;
  const float* head;     // head logits [queries * 64]
  float pre, post;       // weight = ((head * pre) * q_scale) * post
};

// Max over the four consecutive lanes of a quad (DPP quad permutes).
__device__ __forceinline__ uint32_t quad_max(uint32_t v) {
  uint32_t o = __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // lane ^ 1
  v = v > o ? v : o;
  o = __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);           // lane ^ 2
  return v > o ? v : o;
}

template <bool kProducer>
__device__ void prologue_floor(int64_t i, int half, const uint16_t* __restrict__ q,
                               const float* __restrict__ weights, const FloorArgs fa,
                               const FloorProducer fp) {
  using namespace logits_core;
  __shared__ __align__(16) uint32_t codes[kHeads][36];  // 144-byte rows: fewer bank conflicts
  __shared__ float folded[kHeads];
  __shared__ uint32_t keys[kPrologueFloorSamples];
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t wave_sums[4];
  __shared__ uint32_t result[4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int group = lane >> 4;
  const int col = lane & 15;
  const int32_t history = (int32_t)fa.history;  // < 2^25 (the launcher checks)
  uint32_t* out = fa.floors + 2 * i + half;
  if (history < kFloorMinVisible) {
    if (tid == 0) *out = 0u;
    return;
  }
  const int n = (int)floor_samples(history, kPrologueFloorSamples) / 2;  // this half's
  const int stride = history / (2 * n);  // >= 2
  const uint32_t rank = floor_rank(n, fa.count, (int64_t)history + i + 1, kPrologueFloorSigmas);
  if (rank > (uint32_t)n) {
    if (tid == 0) *out = 0u;
    return;
  }
  const int groups = n / 16;
  // Sample m of this half is column (2m + half) stride + stride / 2; wave w
  // scores groups w, w + 4, ...
  v8i b[kPrologueFloorBatch];
  float ks[kPrologueFloorBatch];
  auto load_batch = [&](int g0) {
#pragma unroll
    for (int j = 0; j < kPrologueFloorBatch; ++j) {
      const int g = g0 + 4 * j;
      const uint32_t key = (uint32_t)((2 * (g < groups ? 16 * g + col : col) + half) * stride + stride / 2);
      const v4u* src = reinterpret_cast<const v4u*>(fa.keys + key * (uint32_t)kDim + 32u * group);
      const v4u lo = src[0], hi = src[1];
      b[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      ks[j] = fa.key_scales[key];
    }
  };
  // The query loads first; the sample loads after the quantisation.
  uint4 qraw[4];
  {
    const uint4* src = reinterpret_cast<const uint4*>(q + ((i * kHeads + (tid >> 2)) * kDim + 32 * (tid & 3)));
#pragma unroll
    for (int c = 0; c < 4; ++c) qraw[c] = src[c];
  }
  // Quantise the row's heads: thread t takes head t / 4, dims 32 (t % 4) ..
  // + 31 (the row amax over its four threads).
  {
    const int h = tid >> 2, part = tid & 3;
    float v[32];
    uint32_t m = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 raw = qraw[c];
      const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * c + 2 * j] = bf16_to_f32(words[j] & 0xFFFFu);
        v[8 * c + 2 * j + 1] = bf16_to_f32(words[j] >> 16);
      }
    }
    if constexpr (kProducer) {
      // The producer's RoPE on dims [0, 64): dim j < 32 (part 0) pairs with
      // dim j + 32 (part 1, the next lane); each product and sum rounded to
      // fp32, the result to bf16, as the producer's own Q rows.
#pragma clang fp contract(off)
      int64_t trow = fp.rows ? (int64_t)fp.rows[i] : i;
      if (trow < 0 || trow >= fp.table_rows) trow = 0;  // the Q blocks flag it
      const float* trig = fp.cos_sin + trow * 64;
      float other[32];
#pragma unroll
      for (int j = 0; j < 32; ++j)
        other[j] = __uint_as_float((uint32_t)__builtin_amdgcn_mov_dpp(
            (int)__float_as_uint(v[j]), 0xB1, 0xF, 0xF, false));  // lane ^ 1
      if (part < 2) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float4 cs = *reinterpret_cast<const float4*>(trig + 4 * c);
          const float4 sn = *reinterpret_cast<const float4*>(trig + 32 + 4 * c);
          const float cv[4] = {cs.x, cs.y, cs.z, cs.w};
          const float sv[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x = v[4 * c + j] * cv[j];
            const float y = other[4 * c + j] * sv[j];
            v[4 * c + j] = bf16_to_f32(f32_to_bf16(part == 0 ? x - y : x + y));
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const uint32_t a = __float_as_uint(v[j]) & 0x7FFFFFFFu;
      m = m > a ? m : a;
    }
    m = quad_max(m);
    const float scale = scale_from_amax_bits(m, true);
    const float inverse = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float y[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = fminf(fmaxf(v[4 * c + j] * inverse, -448.0f), 448.0f);
      uint32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
      word = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], word, true);
      codes[h][8 * part + c] = word;
    }
    if (part == 0) {
      if constexpr (kProducer) {
#pragma clang fp contract(off)
        folded[h] = ((fp.head[i * kHeads + h] * fp.pre) * scale) * fp.post;
      } else {
        folded[h] = weights[i * kHeads + h] * scale;
      }
    }
  }
  load_batch(wave);
#pragma unroll
  for (int j = 0; j < 8; ++j) hist[8 * tid + j] = 0;
  if (tid < 4) result[tid] = 0;
  __syncthreads();
  v8i qa[4];
  float wv[16];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const v4u lo = *reinterpret_cast<const v4u*>(&codes[16 * t + col][8 * group]);
    const v4u hi = *reinterpret_cast<const v4u*>(&codes[16 * t + col][8 * group + 4]);
    qa[t] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[4 * t + r] = folded[16 * t + 4 * group + r];
  }
  // sum_h w_h max(s_h, 0) of one group: the lane's 16 heads, then the four
  // lane rows (row-swap permutes).
  auto head_sums = [&](const v4f (&acc)[4], int g, float kscale_key) {
    float p = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) p = fmaf(wv[4 * t + r], fmaxf(acc[t][r], 0.0f), p);
    p = fold32(p, p);
    p = fold16(p, p);
    if (group == 0 && g < groups) keys[16 * g + col] = radix_of(p * kscale_key);
  };
  for (int g0 = wave; g0 < groups; g0 += 4 * kPrologueFloorBatch) {
    if (g0 != wave) load_batch(g0);
    v4f prev[4];
#pragma unroll
    for (int j = 0; j < kPrologueFloorBatch; ++j) {
      v4f acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            qa[t], b[j], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
      if (j > 0) head_sums(prev, g0 + 4 * (j - 1), ks[j - 1]);
#pragma unroll
      for (int t = 0; t < 4; ++t) prev[t] = acc[t];
    }
    head_sums(prev, g0 + 4 * (kPrologueFloorBatch - 1), ks[kPrologueFloorBatch - 1]);
  }
  __syncthreads();
  const uint32_t floor = floor_of_samples<256>(keys, n, rank, hist, wave_sums, result);
  if (tid == 0) *out = floor;
}

// The small stages of a layer step in one launch: blocks [0, nq) quantise
// the indexer Q rows and fold their scales into the head weights, blocks
// [nq, nq + nk) quantise the new index-K rows into the resident cache,
// blocks [nq + nk, nq + nk + nt) pack the new KV tokens into the fp8 paged
// cache, and nf more blocks (when floors are asked for; placed first)
// compute the candidate top-k's per-row floors, two blocks per row. All are independent of
// each other.
__global__ __launch_bounds__(256, kPrologueBlocksPerCu) void layer_prologue(
    const uint16_t* __restrict__ q, int64_t q_rows, const float* __restrict__ weights,
    uint8_t* __restrict__ q_codes, float* __restrict__ q_scales, float* __restrict__ w_folded,
    float* __restrict__ q_fold, const uint16_t* __restrict__ k, int64_t k_rows,
    uint8_t* __restrict__ k_codes,
    float* __restrict__ k_scales, const uint16_t* __restrict__ kv, int64_t tokens,
    int64_t token_offset, const int32_t* __restrict__ page_table, int64_t pages,
    uint8_t* __restrict__ cache, int32_t* __restrict__ status, int64_t nq, int64_t nk,
    int64_t nf, FloorArgs fa) {
  // The floor blocks (the longest) come first in the grid, so that they
  // start at once and the short blocks fill the CUs around them.
  if ((int64_t)blockIdx.x < nf) {
    prologue_floor<false>(blockIdx.x >> 1, (int)(blockIdx.x & 1), q, weights, fa, FloorProducer{});
    return;
  }
  const int64_t b = blockIdx.x - nf;
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
  return dsa_layer_prologue_floors_fp8(q, q_rows, weights, q_codes, q_scales, w_folded, q_fold, k,
                                       k_rows, k_codes, k_scales, kv, tokens, token_offset,
                                       page_table, pages, cache, status, nullptr, nullptr, 0, 0,
                                       nullptr, stream);
}

extern "C" int dsa_layer_prologue_floors_fp8(
    const void* q, int64_t q_rows, const float* weights, void* q_codes, float* q_scales,
    float* w_folded, float* q_fold, const void* k, int64_t k_rows, void* k_codes,
    float* k_scales, const void* kv, int64_t tokens, int64_t token_offset,
    const int32_t* page_table, int64_t pages, void* cache, int32_t* status,
    const void* key_cache, const float* key_cache_scales, int64_t history, int64_t topk,
    uint32_t* floors, hipStream_t stream) {
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
  // Floor blocks: one per query row (q_rows / 64 queries).
  int64_t nf = 0;
  if (floors != nullptr) {
    DSA_CHECK_ARG(q_rows % 64 == 0 && key_cache && key_cache_scales && history >= 0 &&
                      topk >= 1 && topk <= 2048 &&
                      reinterpret_cast<uintptr_t>(key_cache) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(floors) % 4 == 0,
                  "floors need whole queries, the resident key cache (16-byte aligned) and "
                  "k in [1, 2048]");
    DSA_CHECK_ARG(history < ((int64_t)1 << 25), "the key cache must be addressable with 32-bit offsets");
    nf = 2 * (q_rows / 64);  // two per query row
  }
  if (nq + nk + nt + nf == 0) return kOk;
  DSA_CHECK_ARG(nq + nk + nt + nf < 0x7FFFFFFF, "prologue too large for one launch");
  const int64_t columns = history + q_rows / 64;
  const FloorArgs fa{static_cast<const uint8_t*>(key_cache), key_cache_scales, history,
                     (int)(topk < columns ? topk : columns), floors};
  hipLaunchKernelGGL(layer_prologue, dim3((unsigned)(nq + nk + nt + nf)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(q), q_rows, weights,
                     static_cast<uint8_t*>(q_codes), q_scales, w_folded, q_rows ? q_fold : nullptr,
                     static_cast<const uint16_t*>(k), k_rows, static_cast<uint8_t*>(k_codes),
                     k_scales, static_cast<const uint16_t*>(kv), tokens, token_offset, page_table,
                     pages, static_cast<uint8_t*>(cache), status, nq, nk, nf, fa);
  DSA_CHECK_LAUNCH("layer prologue");
  return kOk;
}

namespace dsa {
namespace {

// Indexer input producers: the indexer half of the reference's projection
// step after its two GEMMs (models/deepseek_v32/projections.py:114-121,
// 236-244; rotary.py:47-56). Index K rows get LayerNorm (fp32, rounded to
// bf16), both index Q and index K rows get the non-interleaved RoPE on dims
// [0, 64) (dim i pairs with dim i + 32; real = a cos - b sin, imag = b cos +
// a sin, every product and sum rounded to fp32, the result to bf16), then the
// A1 quantiser. Contraction into FMAs is off in these functions so that each
// operation rounds as the reference's separate elementwise ops do.
//
// A row of 128 is held by 16 lanes, 8 consecutive values each (lane `part`:
// dims 8 part .. 8 part + 7), as in quantize_rows_d128.

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Sum of a row in a fixed order: each lane's 8 values left to right, then
// pairwise across the 16 lanes at distance 8, 4, 2, 1 (every lane ends with
// the same bits).
__device__ __forceinline__ float row_sum_d128(const float v[8]) {
#pragma clang fp contract(off)
  float s = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) s = s + v[i];
#pragma unroll
  for (int offset = 8; offset > 0; offset >>= 1) s = s + __shfl_xor(s, offset, 16);
  return s;
}

// LayerNorm over the row: mean and variance by row_sum_d128, rstd = 1 /
// sqrt(var + eps) (correctly rounded), y = ((x - mean) rstd) w + b, then bf16.
__device__ __forceinline__ void layer_norm_d128(float v[8], int part, const float* __restrict__ w,
                                                const float* __restrict__ b, float eps) {
#pragma clang fp contract(off)
  const float mean = row_sum_d128(v) * 0.0078125f;
  float d[8], sq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    d[i] = v[i] - mean;
    sq[i] = d[i] * d[i];
  }
  const float var = row_sum_d128(sq) * 0.0078125f;
  const float rstd = 1.0f / __builtin_sqrtf(var + eps);
  const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * part);
  const float4 w1 = *reinterpret_cast<const float4*>(w + 8 * part + 4);
  const float4 b0 = *reinterpret_cast<const float4*>(b + 8 * part);
  const float4 b1 = *reinterpret_cast<const float4*>(b + 8 * part + 4);
  const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  const float bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = round_bf16((d[i] * rstd) * ws[i] + bs[i]);
}

// Non-interleaved RoPE on dims [0, 64): dim i < 32 (lanes 0-3) pairs with
// dim i + 32 (lanes 4-7, same slot, lane part ^ 4). `trig`: the token's row
// of the table, cos of the 32 angles then their sin (16-byte aligned).
__device__ __forceinline__ void rope_d128(float v[8], int part, const float* __restrict__ trig) {
#pragma clang fp contract(off)
  float other[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) other[i] = __shfl_xor(v[i], 4, 16);
  if (part < 8) {
    const int d0 = 8 * (part & 3);
    const float4 c0 = *reinterpret_cast<const float4*>(trig + d0);
    const float4 c1 = *reinterpret_cast<const float4*>(trig + d0 + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(trig + 32 + d0);
    const float4 s1 = *reinterpret_cast<const float4*>(trig + 36 + d0);
    const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = v[i] * cs[i];
      const float y = other[i] * sn[i];
      v[i] = round_bf16(part < 4 ? x - y : x + y);
    }
  }
}

struct RopeTable {
  const float* cos_sin;   // [table_rows, 64]
  const int32_t* rows;    // table row of each token, or null: token t uses row t
  int64_t table_rows;
};

// One block of 16 produced rows: load, [LayerNorm], RoPE, quantise (UE8M0),
// store codes and scale; for index Q rows (fold_out set) the head weight
// ((head * pre) * scale) * post. `rows_per_token` rows share a RoPE row.
template <bool kLayerNorm>
__device__ __forceinline__ QuantLane produce_rows_d128(
    int64_t block, const uint16_t* __restrict__ x, int64_t rows, int64_t rows_per_token,
    const RopeTable rope, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    float eps, uint8_t* __restrict__ y, float* __restrict__ scales,
    const float* __restrict__ head, float pre, float post, float* __restrict__ fold_out,
    int32_t* __restrict__ status) {
#pragma clang fp contract(off)
  const int64_t row = (block * 256 + threadIdx.x) >> 4;
  const int part = threadIdx.x & 15;
  const bool live = row < rows;
  uint4 raw = make_uint4(0, 0, 0, 0);
  if (live) raw = *reinterpret_cast<const uint4*>(x + row * 128 + part * 8);
  const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(words[i] & 0xFFFFu);
    v[2 * i + 1] = bf16_to_f32(words[i] >> 16);
  }
  if constexpr (kLayerNorm) layer_norm_d128(v, part, ln_w, ln_b, eps);
  const int64_t token = (live ? row : 0) / rows_per_token;
  int64_t trow = rope.rows ? (int64_t)rope.rows[token] : token;
  if (trow < 0 || trow >= rope.table_rows) {
    if (live && part == 0 && status) atomicOr(status, 2);
    trow = 0;
  }
  rope_d128(v, part, rope.cos_sin + trow * 64);

  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t a = __float_as_uint(v[i]) & 0x7FFFFFFFu;
    m = m > a ? m : a;
  }
  m = max_abs_bits_reduce<16>(m);
  if (!live) return QuantLane{0, 0, 0.0f};
  const float scale = scale_from_amax_bits(m, true);
  const float inverse = 1.0f / scale;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= quantize_one(v[i], scale, inverse, true) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= quantize_one(v[4 + i], scale, inverse, true) << (8 * i);
  *reinterpret_cast<uint2*>(y + row * 128 + part * 8) = make_uint2(lo, hi);
  float fold = 0.0f;
  if (fold_out) fold = ((head[row] * pre) * scale) * post;
  if (part == 0) {
    scales[row] = scale;
    if (fold_out) fold_out[row] = fold;
  }
  return QuantLane{lo, hi, fold};
}

// Blocks [0, nf): the candidate top-k's per-row floors (when asked for),
// then [0, nq): index Q rows (RoPE, quantise, weight fold, partial folded
// queries); [nq, nq + nk): index K rows (LayerNorm, RoPE, quantise into the
// resident cache); the rest: new KV tokens into the fp8 paged cache.
__global__ __launch_bounds__(256, kPrologueBlocksPerCu) void index_producer(
    const uint16_t* __restrict__ q, int64_t q_rows, const float* __restrict__ head, float pre,
    float post, uint8_t* __restrict__ q_codes, float* __restrict__ q_scales,
    float* __restrict__ w_folded, float* __restrict__ q_fold, const uint16_t* __restrict__ k,
    int64_t k_rows, const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
    uint8_t* __restrict__ k_codes, float* __restrict__ k_scales, const RopeTable rope,
    const uint16_t* __restrict__ kv, int64_t token_offset, const int32_t* __restrict__ page_table,
    int64_t pages, uint8_t* __restrict__ cache, int32_t* __restrict__ status, int64_t nq,
    int64_t nk, int64_t nf, FloorArgs fa) {
  // Floor blocks first (the longest), two per query, as in layer_prologue.
  if ((int64_t)blockIdx.x < nf) {
    const FloorProducer fp{rope.cos_sin, rope.rows, rope.table_rows, head, pre, post};
    prologue_floor<true>(blockIdx.x >> 1, (int)(blockIdx.x & 1), q, nullptr, fa, fp);
    return;
  }
  const int64_t b = blockIdx.x - nf;
  if (b < nq) {
    const QuantLane mine = produce_rows_d128<false>(b, q, q_rows, 64, rope, nullptr, nullptr, 0.0f,
                                                    q_codes, q_scales, head, pre, post, w_folded,
                                                    status);
    if (q_fold) fold_partial(b, mine, q_fold);
  } else if (b < nq + nk) {
    produce_rows_d128<true>(b - nq, k, k_rows, 1, rope, ln_w, ln_b, eps, k_codes, k_scales,
                            nullptr, 0.0f, 0.0f, nullptr, status);
  } else {
    pack_tokens(b - nq - nk, kv, k_rows, token_offset, page_table, pages, cache, status);
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_index_producer_fp8(
    const void* q_proj, int64_t tokens, const float* head_logits, float head_pre_scale,
    float head_post_scale, const void* k_proj, const float* norm_weight, const float* norm_bias,
    float norm_eps, const float* cos_sin, int64_t table_rows, const int32_t* rope_rows,
    void* q_codes, float* q_scales, float* weights_out, float* q_fold, void* k_codes,
    float* k_scales, const void* kv, int64_t token_offset, const int32_t* page_table,
    int64_t pages, void* cache, int32_t* status, hipStream_t stream) {
  return dsa_index_producer_floors_fp8(q_proj, tokens, head_logits, head_pre_scale,
                                       head_post_scale, k_proj, norm_weight, norm_bias, norm_eps,
                                       cos_sin, table_rows, rope_rows, q_codes, q_scales,
                                       weights_out, q_fold, k_codes, k_scales, kv, token_offset,
                                       page_table, pages, cache, status, nullptr, nullptr, 0, 0,
                                       nullptr, stream);
}

extern "C" int dsa_index_producer_floors_fp8(
    const void* q_proj, int64_t tokens, const float* head_logits, float head_pre_scale,
    float head_post_scale, const void* k_proj, const float* norm_weight, const float* norm_bias,
    float norm_eps, const float* cos_sin, int64_t table_rows, const int32_t* rope_rows,
    void* q_codes, float* q_scales, float* weights_out, float* q_fold, void* k_codes,
    float* k_scales, const void* kv, int64_t token_offset, const int32_t* page_table,
    int64_t pages, void* cache, int32_t* status, const void* key_cache,
    const float* key_cache_scales, int64_t history, int64_t topk, uint32_t* floors,
    hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(tokens >= 0 && table_rows >= 0 && token_offset >= 0 && pages >= 0,
                "invalid producer shape");
  if (tokens == 0) return kOk;
  DSA_CHECK_ARG(tokens < (int64_t)1 << 24, "too many tokens for one producer launch");
  DSA_CHECK_ARG(q_proj && head_logits && k_proj && norm_weight && norm_bias && cos_sin &&
                    q_codes && q_scales && weights_out && k_codes && k_scales,
                "null pointer");
  DSA_CHECK_ARG(table_rows >= 1 && (rope_rows != nullptr || table_rows >= tokens),
                "the RoPE table must hold a row per token");
  DSA_CHECK_ARG(__builtin_isfinite(norm_eps) && norm_eps >= 0.0f, "norm eps must be finite and >= 0");
  const auto aligned = [](const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  DSA_CHECK_ARG(aligned(q_proj, 16) && aligned(k_proj, 16) && aligned(cos_sin, 16) &&
                    aligned(norm_weight, 16) && aligned(norm_bias, 16) && aligned(q_codes, 8) &&
                    aligned(k_codes, 8) && (q_fold == nullptr || aligned(q_fold, 4)),
                "producer inputs, the RoPE table and norm parameters must be 16-byte aligned, "
                "codes 8-byte aligned");
  const bool pack = kv != nullptr;
  if (pack) {
    DSA_CHECK_ARG(page_table && cache, "null page table or cache");
    DSA_CHECK_ARG(token_offset + tokens <= pages * 64, "tokens exceed the paged cache");
    DSA_CHECK_ARG(aligned(kv, 16) && aligned(cache, 16), "kv and cache must be 16-byte aligned");
  }
  const int64_t nq = (tokens * 64 * 16 + 255) / 256;
  const int64_t nk = (tokens * 16 + 255) / 256;
  const int64_t nt = pack ? (tokens + 3) / 4 : 0;
  // Floor blocks: two per query, sampling the resident key cache's first
  // `history` columns (the query at position history + i sees history + i + 1).
  int64_t nf = 0;
  if (floors != nullptr) {
    DSA_CHECK_ARG(key_cache && key_cache_scales && history >= 0 && topk >= 1 && topk <= 2048 &&
                      aligned(key_cache, 16) && aligned(floors, 4),
                  "floors need the resident key cache (16-byte aligned) and k in [1, 2048]");
    DSA_CHECK_ARG(history < ((int64_t)1 << 25), "the key cache must be addressable with 32-bit offsets");
    nf = 2 * tokens;
  }
  const int64_t columns = history + tokens;
  const FloorArgs fa{static_cast<const uint8_t*>(key_cache), key_cache_scales, history,
                     (int)(topk < columns ? topk : columns), floors};
  const RopeTable rope{cos_sin, rope_rows, table_rows};
  hipLaunchKernelGGL(index_producer, dim3((unsigned)(nf + nq + nk + nt)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(q_proj), tokens * 64, head_logits,
                     head_pre_scale, head_post_scale, static_cast<uint8_t*>(q_codes), q_scales,
                     weights_out, q_fold, static_cast<const uint16_t*>(k_proj), tokens,
                     norm_weight, norm_bias, norm_eps, static_cast<uint8_t*>(k_codes), k_scales,
                     rope, static_cast<const uint16_t*>(kv), token_offset, page_table, pages,
                     static_cast<uint8_t*>(cache), status, nq, nk, nf, fa);
  DSA_CHECK_LAUNCH("index producer");
  return kOk;
}
