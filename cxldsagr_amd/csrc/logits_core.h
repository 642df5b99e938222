// Arithmetic of the fp8 indexer logits shared by the logits kernels
// (logits.hip) and the exact row recompute of the candidate top-k
// (topk.hip): one definition, so that a score computed by either kernel has
// the same bits.
//
//   out[i, j] = kscale[j] * sum_{h<64} w[i, h] * relu(sum_{d<128} q[i,h,d] * k[j,d])
//
// (operators/deepseek_v32/indexer/echo.py:339-410). Per (query, 16 keys):
// four v_mfma_f32_16x16x128_f8f6f4 with A = 16 heads x 128 dims of the query
// and B = 128 dims x 16 keys (lane l: head 16t + 4(l/16) + r, key l % 16 in
// register r of tile t), then relu(s) w = (|s| + s) w / 2: the |s| half is
// one fmaf chain per lane over its 16 heads (head_sum), and the linear half
// sum_h (w_h / 2) s_h = k . q' is one more MFMA whose A operand holds
// q' = sum_h (w_h / 2) q_h as four e4m3 digits (query_digits). The four
// 16-lane rows are then summed by reduce_scatter4 so lane l holds key l of a
// 64-key pass. Files that include this header are compiled with the same
// flags (no NaN canonicalisation, VGPR-form MFMA).
#pragma once

#include <utility>

#include "dsa_common.h"

namespace dsa {
namespace logits_core {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kHeads = 64;
constexpr int kDim = 128;
constexpr int kDigits = 4;           // e4m3 digits of the folded query
constexpr int kQueriesPerWave = 2;   // queries whose digits share one A operand

// f(integral_constant<int, I>) for every I of the sequence, in order.
template <typename F, int... I>
__device__ __forceinline__ void for_each_index(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

// Sum of x over lanes l and l ^ 32 (first operand) and of y likewise, with
// the results exchanged so that lanes 0-31 get x's sum and lanes 32-63 y's.
__device__ __forceinline__ float fold32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same for lanes l and l ^ 16: rows 0 and 2 get x's sums, rows 1 and 3 y's.
__device__ __forceinline__ float fold16(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// part[u] holds the row-partial sums for key 16u + l % 16; returns the total
// for key l of the 64-key pass.
__device__ __forceinline__ float reduce_scatter4(const float part[4]) {
  const float a0 = fold32(part[0], part[2]);  // rows 0-1: key group 0, rows 2-3: group 2
  const float a1 = fold32(part[1], part[3]);  // rows 0-1: group 1, rows 2-3: group 3
  return fold16(a0, a1);                      // row g: key group g
}

// The A operand of head tile t (heads 16t .. 16t + 15) of query row qc: lane
// (col, group) holds head 16t + col, dims 32 group .. 32 group + 31.
__device__ __forceinline__ v8i query_operand(const uint8_t* __restrict__ q, int64_t qc, int t,
                                             int col, int group) {
  const v4u* src = reinterpret_cast<const v4u*>(q + ((qc * kHeads + 16 * t + col) * kDim + 32 * group));
  const v4u lo = src[0], hi = src[1];
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// The B operand of 16 keys straight from the key cache: lane (col, group)
// holds dims 32 group .. 32 group + 31 of key `key` (the bytes the logits
// kernel reads from its swizzled LDS stage).
__device__ __forceinline__ v8i key_operand(const uint8_t* __restrict__ k, int64_t key, int group) {
  const v4u* src = reinterpret_cast<const v4u*>(k + key * kDim + 32 * group);
  const v4u lo = src[0], hi = src[1];
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// One lane's share of the head sum for one (query, key): |s| w / 2 over its
// 16 heads in one fmaf chain in head-tile order (wt holds w / 2), plus the
// linear MFMA's share `lin` scaled by `fl`.
__device__ __forceinline__ float head_sum(const v4f (&acc)[4], float lin, const float (&wt)[16],
                                          float fl) {
  float p = fabsf(acc[0][0]) * wt[0];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = (t == 0 ? 1 : 0); r < 4; ++r) p = fmaf(fabsf(acc[t][r]), wt[4 * t + r], p);
  return fmaf(lin, fl, p);
}

// Partial folded queries from the query codes: pg[g][i] = sum over heads
// 16g .. 16g + 15 (increasing) of w_h * q[h, 4c + i], one fmaf chain from 0
// per entry, for lane 32j + c (query j of the wave, dims 4c .. 4c + 3).
// `codes[h]` holds q[h, 4c .. 4c + 3]; `w4` the weights of heads 4m .. 4m + 3
// (m = lane % 16), each broadcast along its 16-lane row by DPP row_newbcast.
// The layer prologue forms the same chains (q_fold).
__device__ __forceinline__ void fold_partials(const uint32_t (&codes)[kHeads], v4f w4, bool live,
                                              float (&pg)[4][4]) {
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) pg[g][i] = 0.0f;
  auto add_head = [&](auto head) {
    constexpr int h = decltype(head)::value;
    const float wb = __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(w4[h & 3]), 0x150 + (h >> 2), 0xF, 0xF, false));
    const float wh = live ? wb : 0.0f;
    const v2f x0 = __builtin_amdgcn_cvt_pk_f32_fp8(codes[h], false);
    const v2f x1 = __builtin_amdgcn_cvt_pk_f32_fp8(codes[h], true);
    float* p = pg[h >> 4];
    p[0] = fmaf(wh, x0[0], p[0]);
    p[1] = fmaf(wh, x0[1], p[1]);
    p[2] = fmaf(wh, x1[0], p[2]);
    p[3] = fmaf(wh, x1[1], p[3]);
  };
  for_each_index(add_head, std::make_integer_sequence<int, kHeads>{});
}

// The linear MFMA's A operand for the two queries of a wave from their
// partial folded queries (lane 32j + c: query j, dims 4c .. 4c + 3):
// q' = 0.5 (((p0 + p1) + p2) + p3) is written as kDigits e4m3 digits, digit
// d at scale 2^(E_j - 4d) (|q'| < 2^(E_j + 8)), each the residual of the
// ones before it to half an e4m3 ulp. Row 4d + j of the operand is digit d
// of query j (rows of j >= 2 are zero), so its C row lands in lane group d,
// register j, and the reduction over lane groups also sums the digits.
// `digits` is the wave's own LDS scratch [2][kDigits][kDim]; fl[r] receives
// the scale of query r's C row in this lane's group.
__device__ __forceinline__ void query_digits(const float (&pg)[4][4],
                                             uint8_t (*digits)[kDigits][kDim], int lane,
                                             v8i& qd, float (&fl)[kQueriesPerWave]) {
  static_assert(kQueriesPerWave == 2, "the fold maps 32 lanes x 4 dims to a query");
  const int j = lane >> 5;
  const int c = lane & 31;
  const int group = lane >> 4;
  float qp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qp[i] = 0.5f * (((pg[0][i] + pg[1][i]) + pg[2][i]) + pg[3][i]);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(qp[i]));
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
  int ex = 0;
  (void)frexpf(amax, &ex);  // amax < 2^ex (ex = 0 for amax = 0)
  const int e0 = ex - 8;
#pragma unroll
  for (int d = 0; d < kDigits; ++d) {
    const int e = e0 - 4 * d;
    uint32_t code = 0;
    code = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(qp[0], -e), ldexpf(qp[1], -e), code, false);
    code = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(qp[2], -e), ldexpf(qp[3], -e), code, true);
    *reinterpret_cast<uint32_t*>(&digits[j][d][4 * c]) = code;
    const v2f y0 = __builtin_amdgcn_cvt_pk_f32_fp8(code, false);
    const v2f y1 = __builtin_amdgcn_cvt_pk_f32_fp8(code, true);
    qp[0] -= ldexpf(y0[0], e);
    qp[1] -= ldexpf(y0[1], e);
    qp[2] -= ldexpf(y1[0], e);
    qp[3] -= ldexpf(y1[1], e);
  }
  // A operand: lane l holds row l % 16 = 4d + j', dims 32 (l / 16) .. + 31;
  // rows j' >= 2 (no query) are zero.
  const int jr = lane & 3, dr = (lane & 15) >> 2, blk = lane >> 4;
  const bool jlive = jr < kQueriesPerWave;
  const int jc = jlive ? jr : 0;
  v4u lo = *reinterpret_cast<const v4u*>(&digits[jc][dr][32 * blk]);
  v4u hi = *reinterpret_cast<const v4u*>(&digits[jc][dr][32 * blk + 16]);
  if (!jlive) lo = hi = v4u{0u, 0u, 0u, 0u};
  qd = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  // C rows of lane group g = digit g: register r (query r) is scaled by
  // 2^(E_r - 4g).
#pragma unroll
  for (int r = 0; r < kQueriesPerWave; ++r)
    fl[r] = ldexpf(1.0f, __builtin_amdgcn_readlane(e0, 32 * r) - 4 * group);
}

// Order-preserving 32-bit key of an fp32 value (descending key = descending
// value, -0.0 below +0.0, NaN by its bits), as the top-k defines it.
__device__ __forceinline__ uint32_t radix_of(float v) {
  const uint32_t b = __float_as_uint(v);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

// ---- per-row floors of the candidate top-k (the sample and its rank).
//
// A floor F (a radix key) such that, with overwhelming probability, the row
// has at least `count` scores at or above it, so that the scores at or above
// F contain the row's top `count`; the top-k checks this exactly and
// recomputes a row whose floor was too high. F is estimated from the row's
// own scores at n evenly spaced sample columns (a multiple of 64, at least
// kFloorMinSamples, about 1/64 of the columns sampled, at most the caller's
// maximum): with E = n count / visible the expected number of samples in the
// top `count`, F is the r-th largest sample score for r = E + 6 sqrt(E) + 2
// (to two radix digits, so F is at or below it), about 6 sigma above E, and
// the scores at or above F are about (r / n) visible (~4.2K per row at 64K
// columns). Rows of fewer than kFloorMinVisible visible columns get F = 0
// (selected from their full scores), as do rows whose estimate falls at or
// below the radix key of -inf. The sample scores need not have the bits of
// the logits kernel (F is an estimate); they use the plain formula on the
// same MFMA dot products.
constexpr int kFloorMinSamples = 1024;
constexpr int kFloorMaxSamples = 4096;
constexpr int64_t kFloorMinVisible = 8192;
constexpr uint32_t kFloorNegInfKey = 0x007FFFFFu;

// Samples for `span` columns (at most `max_samples`).
__device__ __forceinline__ int64_t floor_samples(int64_t span, int64_t max_samples) {
  int64_t n = (span / 64) & ~(int64_t)63;
  return n < kFloorMinSamples ? kFloorMinSamples : n > max_samples ? max_samples : n;
}

__device__ __forceinline__ uint32_t floor_rank(int64_t n, int count, int64_t visible,
                                               float sigmas = 6.0f) {
  const float expected = (float)n * (float)count / (float)visible;
  return (uint32_t)ceilf(expected + sigmas * sqrtf(expected)) + 2u;
}

// A row's floor is kept as two estimates, floors[2 row] and floors[2 row + 1]
// (from disjoint halves of its sample, or the same value twice), and is
// their minimum: it is too high only when both are. 0 = no floor (the row is
// selected from its full scores).
__device__ __forceinline__ uint32_t row_floor(const uint32_t* __restrict__ floors, int64_t row) {
  const uint32_t a = floors[2 * row], b = floors[2 * row + 1];
  return a < b ? a : b;
}

// Radix select in LDS by a work-group of kBlock threads: the digit d (of
// `width` bits at `shift`) of the `rank`-th largest of the n keys whose bits
// above shift + width equal `prefix` (hist has 2048 entries, zero on entry
// and on exit). Returns the digit and reduces `rank` to the rank inside it.
// Inclusive suffix sum over the wave (lane l: the sum over lanes >= l) with
// VALU lane moves: DPP row shifts inside each 16-lane row, then the totals of
// the higher rows.
__device__ __forceinline__ uint32_t wave_suffix_sum(uint32_t v) {
  const int lane = threadIdx.x & 63;
  // row_shl:k (0x100 + k): lane l reads lane l + k of its row, 0 past the row.
  v += __builtin_amdgcn_update_dpp(0u, v, 0x101, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0u, v, 0x102, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0u, v, 0x104, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0u, v, 0x108, 0xF, 0xF, false);
  const uint32_t r1 = __builtin_amdgcn_readlane(v, 16), r2 = __builtin_amdgcn_readlane(v, 32),
                 r3 = __builtin_amdgcn_readlane(v, 48);
  const int row = lane >> 4;
  return v + (row < 1 ? r1 : 0u) + (row < 2 ? r2 : 0u) + (row < 3 ? r3 : 0u);
}

template <int kBlock>
__device__ uint32_t floor_digit(const uint32_t* __restrict__ keys, int n, uint32_t prefix,
                                int shift, int width, uint32_t* __restrict__ hist,
                                uint32_t* __restrict__ wave_sums, uint32_t* __restrict__ result,
                                uint32_t& rank) {
  constexpr int kPer = 2048 / kBlock;
  constexpr int kWavesB = kBlock / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t mask = (1u << width) - 1u;
  const int hi = shift + width;
  for (int i = tid; i < n; i += kBlock) {
    const uint32_t key = keys[i];
    const bool in = hi >= 32 || (key >> hi) == prefix;
    if (in) atomicAdd(&hist[(key >> shift) & mask], 1u);
  }
  __syncthreads();
  // Thread t owns bins kPer t .. kPer t + kPer - 1; suffix counts from the top.
  uint32_t c[kPer], own = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    c[j] = hist[kPer * tid + j];
    own += c[j];
  }
  const uint32_t incl = wave_suffix_sum(own);  // this thread's and the higher threads' bins
  if (lane == 0) wave_sums[wave] = incl;
  __syncthreads();
  uint32_t above = incl - own;
  for (int w = wave + 1; w < kWavesB; ++w) above += wave_sums[w];
#pragma unroll
  for (int j = kPer - 1; j >= 0; --j) {
    if (c[j] && above < rank && above + c[j] >= rank) {
      result[0] = kPer * tid + j;
      result[1] = rank - above;
    }
    above += c[j];
    hist[kPer * tid + j] = 0;
  }
  __syncthreads();
  const uint32_t d = result[0];
  rank = result[1];
  return d;
}

// The floor from n sample radix keys in LDS (hist zero on entry and exit):
// the rank-th largest key to two 11-bit digits (below it by less than 2^10
// in radix order); 0 at or below the radix key of -inf.
template <int kBlock>
__device__ __forceinline__ uint32_t floor_of_samples(const uint32_t* __restrict__ keys, int n,
                                                     uint32_t rank, uint32_t* __restrict__ hist,
                                                     uint32_t* __restrict__ wave_sums,
                                                     uint32_t* __restrict__ result) {
  uint32_t r = rank;
  const uint32_t d1 = floor_digit<kBlock>(keys, n, 0u, 21, 11, hist, wave_sums, result, r);
  const uint32_t d2 = floor_digit<kBlock>(keys, n, d1, 10, 11, hist, wave_sums, result, r);
  const uint32_t floor = (d1 << 21) | (d2 << 10);
  return floor > kFloorNegInfKey ? floor : 0u;
}

// The scores of one query row for every column in [0, columns) into out_row,
// with the arithmetic of the logits kernel (same operands, same MFMAs, same
// epilogue order), so each score has the bits that kernel gives it. Called
// by every wave of a work-group (same arguments): wave `wave` of `waves`
// computes the 64-column passes wave, wave + waves, ... Columns outside
// [qs, qe) are -inf. `digits` is this wave's LDS scratch. A slow path: B
// operands come straight from memory and each wave keeps one query.
__device__ __forceinline__ void row_scores(const uint8_t* __restrict__ q,
                                           const uint8_t* __restrict__ k,
                                           const float* __restrict__ w,
                                           const float* __restrict__ kscale,
                                           const float* __restrict__ q_fold, int64_t row,
                                           int32_t qs, int32_t qe, int64_t columns,
                                           float* __restrict__ out_row,
                                           uint8_t (*digits)[kDigits][kDim], int wave, int waves) {
  const int lane = threadIdx.x & 63;
  const int group = lane >> 4;
  const int col = lane & 15;
  // This wave's query 0 is the row; query 1 is empty (zero digits, zero
  // weights). The MFMA rows of query 0 do not depend on query 1's.
  const bool flive = (lane >> 5) == 0;
  const int fc = lane & 31;
  float pg[4][4];
  if (q_fold) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v4f a = *reinterpret_cast<const v4f*>(q_fold + (row * 4 + g) * kDim + 4 * fc);
#pragma unroll
      for (int i = 0; i < 4; ++i) pg[g][i] = flive ? a[i] : 0.0f;
    }
  } else {
    uint32_t codes[kHeads];
    const uint8_t* qrow = q + row * kHeads * kDim + 4 * fc;
#pragma unroll
    for (int h = 0; h < kHeads; ++h) codes[h] = *reinterpret_cast<const uint32_t*>(qrow + h * kDim);
    const v4f w4 = *reinterpret_cast<const v4f*>(w + row * kHeads + 4 * (fc & 15));
    fold_partials(codes, w4, flive, pg);
  }
  v8i qd;
  float fl[kQueriesPerWave];
  query_digits(pg, digits, lane, qd, fl);
  v8i qa[4];
  float wt[16];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    qa[t] = query_operand(q, row, t, col, group);
    const v4f wv = *reinterpret_cast<const v4f*>(w + row * kHeads + 16 * t + 4 * group);
#pragma unroll
    for (int r = 0; r < 4; ++r) wt[4 * t + r] = 0.5f * wv[r];
  }
  const int64_t passes = (columns + 63) / 64;
  for (int64_t p = wave; p < passes; p += waves) {
    float part[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      int64_t key = 64 * p + 16 * u + col;
      if (key > columns - 1) key = columns - 1;  // past the end: the column is not stored
      const v8i b = key_operand(k, key, group);
      v4f acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[t], b, v4f{0.0f, 0.0f, 0.0f, 0.0f},
                                                                  0, 0, 0, 0, 0, 0);
      const v4f lin = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
          qd, b, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
      part[u] = head_sum(acc, lin[0], wt, fl[0]);
    }
    const float total = reduce_scatter4(part);
    const int64_t key = 64 * p + lane;
    if (key < columns) {
      const bool visible = key >= qs && key < qe;
      out_row[key] = visible ? total * kscale[key] : -__builtin_inff();
    }
  }
}

}  // namespace logits_core
}  // namespace dsa
