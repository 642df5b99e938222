// A4: fp8 MQA indexer logits on CDNA4 MFMA with the causal -inf tail fused.
//
//   out[i, j] = kscale[j] * sum_{h<64} w[i, h] * relu(sum_{d<128} q[i,h,d] * k[j,d])
//
// for starts[i] <= j < ends[i]; -inf elsewhere, including the padded columns
// [columns, ldo). Semantics: operators/deepseek_v32/indexer/echo.py:339-410
// (resident branch) with the tail mask of echo.py:224-249 fused in.
//
// Mapping (gfx950, wave64):
// * v_mfma_f32_16x16x128_f8f6f4 with A = 16 heads x 128 dims of one query
//   (resident in VGPRs for the whole key loop) and B = 128 dims x 16 keys
//   read from LDS; one instruction is a full 128-deep dot product.
// * C layout: lane l, register r -> head 16t + 4(l/16) + r, key l%16. The
//   head-weighted ReLU sum uses relu(s) = (s + |s|) / 2: the |s| half is 16
//   in-lane FMAs per key per query (|s| is a free source modifier), and the
//   linear half, sum_h w_h s_h / 2 = k . q' with q' = sum_h w_h q_h / 2, is
//   one more MFMA per 16 keys for both queries of a wave, with q' held as
//   four e4m3 digits (q' to ~2^-17 of its largest element). The four lane
//   rows are then combined with a reduce-scatter on the gfx950 row-swap
//   permutes (v_permlane32_swap, v_permlane16_swap) so lane l ends with key
//   l of a 64-key pass: one coalesced 256-byte row store.
// * The epilogue of one (query, 16-key) unit runs while the four MFMAs of the
//   next unit execute (explicitly interleaved).
// * Work-group: 8 waves (two per SIMD) x 2 queries = 16 queries; the key
//   range is split so the grid is about one work-group per CU. Q of a wave's
//   two queries stays in registers (under 256 VGPRs, so two waves fit a
//   SIMD) and each B operand read from LDS feeds 9 MFMAs. With one wave per
//   SIMD the MFMA pipe idles while the wave runs its epilogue and row tail;
//   the second wave issues MFMAs in those gaps.
// * K stages (128 keys x 128 B, plus the 128 key scales) arrive by LDS DMA
//   (global_load_lds_dwordx4 / _dword) into a ring kRing - 1 stages ahead,
//   with the 16-byte chunks of each key XOR-swizzled by (key & 7) against
//   bank conflicts of the B-operand reads; one barrier per stage, and the
//   stage is computed in two passes of 64 keys.
// * Loads and stores never share a wave: vmcnt counts both, and with stores
//   pending it no longer says which loads are done. Wave 0 issues every DMA
//   (and waits on vmcnt for them) but stores nothing; its rows go through LDS
//   to waves 1-7, which store their own rows and wave 0's in turn.
#include <utility>

#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kHeads = 64;
constexpr int kDim = 128;
constexpr int kWaves = 8;
constexpr int kQueriesPerWave = 2;
constexpr int kQueriesPerBlock = kWaves * kQueriesPerWave;
constexpr int kStageKeys = 128;                    // keys per DMA stage and barrier
constexpr int kHalfKeys = 64;                      // keys per compute pass (lane = key)
constexpr int kThreads = kWaves * 64;
constexpr int kRing = 4;
constexpr int kKBytes = kStageKeys * kDim;         // 16 KB of keys per stage
constexpr int kKLoads = kKBytes / (64 * 16);       // DMA instructions for the keys (wave 0)
constexpr int kSLoads = kStageKeys / 64;           // DMA instructions for the key scales
constexpr int kStageBytes = kKBytes + kStageKeys * 4;  // + the stage's key scales
constexpr int kDigits = 4;                         // e4m3 digits of the folded query
// Radix-digit counts for the top-k (optional output): per query row, the
// number of its scores in [0, columns) by the top 11 bits of their radix key
// (the top-k's level-0 digit). A work-group counts its rows in LDS as two
// 16-bit counters per word - digit d in half d >> 10 of word d & 1023, so
// neighbouring digits (the crowded ones) sit in different words - and adds
// the nonzero ones to the global counts at the end. A split covers at most
// kMaxSplitKeys keys, so a counter cannot carry into its neighbour.
constexpr int kDigitBins = 2048;
constexpr int kDigitShift = 21;
constexpr int64_t kMaxSplitKeys = 65535 / kStageKeys * kStageKeys;
constexpr uint32_t kNegInfDigit = 0x007FFFFFu >> kDigitShift;  // radix key of -inf, top 11 bits

// The count word and half of a score's digit, d = radix(v) >> 21: for v >= 0
// (sign clear) d = 1024 + bits 21-30 of v, for v < 0 d = 1023 - bits 21-30,
// so the word d & 1023 is those bits, flipped when the sign is set, and the
// half d >> 10 is the sign's complement.
__device__ __forceinline__ uint32_t digit_word(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t flip = (uint32_t)((int32_t)b >> 31) & 1023u;
  return ((b >> kDigitShift) & 1023u) ^ flip;
}
__device__ __forceinline__ uint32_t digit_half_shift(float v) {
  return (~__float_as_uint(v) >> 27) & 16u;  // 16 for the upper half
}


// f(integral_constant<int, I>) for every I of the sequence, in order.
template <typename F, int... I>
__device__ __forceinline__ void for_each_index(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

__device__ __forceinline__ v4u lds_v4u(uint32_t addr) {
  return *(const v4u __attribute__((address_space(3)))*)(uintptr_t)addr;
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int kOutstanding>
__device__ __forceinline__ void wait_dma() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kOutstanding) : "memory");
}

// LDS DMA, scalar base: 16 or 4 bytes per lane from base + off (32-bit lane
// offset) to lds_base + 16 l or + 4 l.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               ::"s"(lds_base), "v"(off), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void dma4_s(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               ::"s"(lds_base), "v"(off), "s"(base) : "memory", "m0");
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
// for key l of the stage.
__device__ __forceinline__ float reduce_scatter4(const float part[4]) {
  const float a0 = fold32(part[0], part[2]);  // rows 0-1: key group 0, rows 2-3: group 2
  const float a1 = fold32(part[1], part[3]);  // rows 0-1: group 1, rows 2-3: group 3
  return fold16(a0, a1);                      // row g: key group g
}

template <bool kCount>
__global__ __launch_bounds__(kThreads, 1) void logits_fp8_mfma(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ k, const float* __restrict__ w,
    const float* __restrict__ kscale, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ ends, int64_t query_start, int64_t rows, int64_t columns,
    int64_t ldo, int64_t keys_per_split, const float* __restrict__ q_fold, float* __restrict__ out,
    uint32_t* __restrict__ digit_counts) {
  __shared__ __align__(16) uint8_t ring[kRing][kStageBytes];
  // Packed 16-bit digit counts of the block's rows: digit d of row i is half
  // d >> 10 of word i * kDigitBins / 2 + (d & 1023).
  constexpr int kBinWords = kQueriesPerBlock * kDigitBins / 2;
  constexpr int kBinVecs = kBinWords / (4 * kThreads);  // 16-byte LDS accesses per thread
  __shared__ __align__(16) uint32_t bins[kCount ? kBinWords : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int group = lane >> 4;
  const int col = lane & 15;
  const int64_t q0 = (int64_t)blockIdx.y * kQueriesPerBlock;
  const int64_t kb = (int64_t)blockIdx.x * keys_per_split;
  if (kb >= ldo) return;  // a padding split (whole work-group, before any barrier)
  const int64_t ke = kb + keys_per_split < ldo ? kb + keys_per_split : ldo;
  const float neg_inf = -__builtin_inff();
  // Keys of this split that the digit counts cover.
  const int64_t count_end = ke < columns ? ke : columns;
  if constexpr (kCount) {
    // Ordered before the first count by the first stage's barrier (or the
    // barrier before the flush when there are no stages).
#pragma unroll
    for (int i = 0; i < kBinVecs; ++i)
      reinterpret_cast<v4u*>(bins)[i * kThreads + tid] = v4u{0u, 0u, 0u, 0u};
  }

  // Largest causal end among this block's queries: keys at or beyond it
  // are -inf for every row and need no MFMA work.
  int64_t max_end = 0;
  for (int i = 0; i < kQueriesPerBlock; ++i) {
    const int64_t qi = q0 + i;
    if (qi < rows) {
      const int64_t e = ends ? (int64_t)ends[qi] : query_start + qi + 1;
      max_end = e > max_end ? e : max_end;
    }
  }
  if (max_end > columns) max_end = columns;
  const int64_t kend = ke < max_end ? ke : max_end;
  const int stages = kend > kb ? (int)((kend - kb + kStageKeys - 1) / kStageKeys) : 0;

  // DMA plan (wave 0 only): K chunk p = 64 i + lane of a stage (load i) is
  // key 8i + lane / 8, stored chunk lane % 8 = logical chunk ^ (key & 7); then
  // 4-byte loads of the stage's key scales (key 64 i + lane). Keys past the
  // end re-read the last key (their columns are -inf), and stages past the
  // end key 0.
  const uint32_t ring_base = (uint32_t)(uintptr_t)&ring[0][0];
  const int lane_key = lane >> 3;
  const uint32_t lane_chunk = 16u * (uint32_t)((lane & 7) ^ (lane_key & 7));
  const uint32_t lane_off = (uint32_t)lane_key * kDim + lane_chunk;
  auto issue = [&](int s) {
    const uint32_t slot_base = ring_base + (uint32_t)(s % kRing) * kStageBytes;
    const bool live = s < stages;
    const int64_t key0 = live ? kb + (int64_t)s * kStageKeys : 0;
    const int32_t last = live ? (int32_t)(columns - 1 - key0) : 0;  // >= 0: key0 < columns
    const uint8_t* kbase = k + key0 * kDim;
    if (last >= kStageKeys - 1) {
      // A whole stage: every lane offset is a constant and the per-load
      // steps go into the scalar base (no vector arithmetic per load).
#pragma unroll
      for (int i = 0; i < kKLoads; ++i) dma16_s(kbase + 1024 * i, lane_off, slot_base + i * 1024);
#pragma unroll
      for (int i = 0; i < kSLoads; ++i)
        dma4_s(kscale + key0 + 64 * i, 4u * (uint32_t)lane, slot_base + kKBytes + 256 * i);
    } else {
#pragma unroll
      for (int i = 0; i < kKLoads; ++i) {
        const int32_t key = min(8 * i + lane_key, last);
        dma16_s(kbase, (uint32_t)key * kDim + lane_chunk, slot_base + i * 1024);
      }
#pragma unroll
      for (int i = 0; i < kSLoads; ++i)
        dma4_s(kscale + key0, 4u * (uint32_t)min(64 * i + lane, last), slot_base + kKBytes + 256 * i);
    }
  };
  // The first stages' keys are on their way while the query operands load
  // (wave 0's loads complete in issue order, the DMA first).
  if (wave == 0) {
#pragma unroll
    for (int s = 0; s < kRing - 1; ++s) issue(s);
  }


  // Per-wave query operands and head weights (lane rows: heads 16t + 4g + r).
  // Key positions fit int32 (the launcher checks ldo < 2^31).
  v8i qa[kQueriesPerWave][4];
  float wt[kQueriesPerWave][16];
  int32_t qs[kQueriesPerWave], qe[kQueriesPerWave];
  const int64_t qw = q0 + wave * kQueriesPerWave;

  // Linear half of the head sum: sum_h (w_h / 2) s_h = k . q' with
  // q' = sum_h (w_h / 2) q_h, formed here in fp32 (lane 32j + c: query j,
  // dims 4c .. 4c + 3) and written as kDigits e4m3 digits, digit d at scale
  // 2^(E_j - 4d) (|q'| < 2^(E_j + 8)): each digit holds the residual of the
  // ones before it to within half an e4m3 ulp, so the four carry q' to about
  // 2^-17 of its largest element. In the MFMA operand, row 4d + j is digit d
  // of query j (rows 4d + 2 and 4d + 3 are zero); its C row then sits in lane
  // group d, register j, so the reduction over lane groups that sums head
  // partials also sums the digits.
  //
  // Load order: the inputs of q' and the head weights first, then the query
  // operands (the bulk of the bytes), so that forming q' waits only for its
  // own inputs and overlaps the latency of the query operands.
  __shared__ __align__(16) uint8_t digits[kWaves][kQueriesPerWave][kDigits][kDim];
  v8i qd;
  float fl[kQueriesPerWave];
  static_assert(kQueriesPerWave == 2, "the fold maps 32 lanes x 4 dims to a query");
  const int fj = lane >> 5;
  const int fc = lane & 31;
  const bool flive = qw + fj < rows;
  const int64_t fqc = flive ? qw + fj : 0;
  // q' in four partial sums over heads 16g .. 16g + 15 (each one fmaf chain
  // from 0 in increasing head order), then 0.5 (((p0 + p1) + p2) + p3): the
  // same bits whether the partials come from the layer prologue (q_fold,
  // [rows][4][128]) or are formed here.
  float pg[4][4];
  uint32_t codes[kHeads];
  v4f w4;
  if (q_fold) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v4f a = *reinterpret_cast<const v4f*>(q_fold + (fqc * 4 + g) * kDim + 4 * fc);
#pragma unroll
      for (int i = 0; i < 4; ++i) pg[g][i] = flive ? a[i] : 0.0f;
    }
  } else {
    // All 64 heads' codes in flight at once; the weights of heads 4m ..
    // 4m + 3 per lane (m = lane % 16, the lane's place in its 16-lane row).
    const uint8_t* qrow = q + fqc * kHeads * kDim + 4 * fc;
#pragma unroll
    for (int h = 0; h < kHeads; ++h) codes[h] = *reinterpret_cast<const uint32_t*>(qrow + h * kDim);
    w4 = *reinterpret_cast<const v4f*>(w + fqc * kHeads + 4 * (fc & 15));
  }
#pragma unroll
  for (int j = 0; j < kQueriesPerWave; ++j) {
    const int64_t qi = qw + j;
    const bool live = qi < rows;
    const int64_t qc = live ? qi : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const v4f wv = *reinterpret_cast<const v4f*>(w + qc * kHeads + 16 * t + 4 * group);
#pragma unroll
      for (int r = 0; r < 4; ++r) wt[j][4 * t + r] = live ? 0.5f * wv[r] : 0.0f;
    }
    // A dead query gets an empty visible range; its stores are skipped anyway.
    int64_t e = ends ? (int64_t)ends[qc] : query_start + qc + 1;
    if (e > columns) e = columns;
    qs[j] = live ? (starts ? starts[qc] : 0) : 0;
    qe[j] = live ? (int32_t)e : 0;
  }
#pragma unroll
  for (int j = 0; j < kQueriesPerWave; ++j) {
    const int64_t qc = qw + j < rows ? qw + j : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const v4u* src = reinterpret_cast<const v4u*>(q + ((qc * kHeads + 16 * t + col) * kDim + 32 * group));
      const v4u lo = src[0], hi = src[1];
      qa[j][t] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
  }
  {
    const int j = fj;
    const int c = fc;
    if (!q_fold) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) pg[g][i] = 0.0f;
      // Each head's weight broadcast along the 16-lane row by DPP
      // (row_newbcast).
      auto add_head = [&](auto head) {
        constexpr int h = decltype(head)::value;
        const float wb = __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(w4[h & 3]), 0x150 + (h >> 2), 0xF, 0xF, false));
        const float wh = flive ? wb : 0.0f;
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
      *reinterpret_cast<uint32_t*>(&digits[wave][j][d][4 * c]) = code;
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
    v4u lo = *reinterpret_cast<const v4u*>(&digits[wave][jc][dr][32 * blk]);
    v4u hi = *reinterpret_cast<const v4u*>(&digits[wave][jc][dr][32 * blk + 16]);
    if (!jlive) lo = hi = v4u{0u, 0u, 0u, 0u};
    qd = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    // C rows of lane group g = digit g: register r (query r) is scaled by
    // 2^(E_r - 4g).
#pragma unroll
    for (int r = 0; r < kQueriesPerWave; ++r)
      fl[r] = ldexpf(1.0f, __builtin_amdgcn_readlane(e0, 32 * r) - 4 * group);
  }

  // Wave 0's finished rows, [stage parity][query][key].
  __shared__ __align__(16) float staged[2][kQueriesPerWave][kStageKeys];
  auto store_staged = [&](int st) {
#pragma unroll
    for (int hf = 0; hf < kStageKeys / kHalfKeys; ++hf) {
      const int64_t key = kb + (int64_t)st * kStageKeys + kHalfKeys * hf + lane;
#pragma unroll
      for (int j = 0; j < kQueriesPerWave; ++j) {
        const int64_t qi = q0 + j;  // wave 0's queries
        if (qi < rows && key < ke) out[qi * ldo + key] = staged[st & 1][j][kHalfKeys * hf + lane];
      }
    }
  };

  // All compiler-visible global loads (and the first stages' DMA) complete
  // here: from now on wave 0's vmcnt counts DMA only.
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // Digit counts of the previous half-stage's scores, issued under the next
  // half-stage's MFMAs (lane bit j of pend_ok: query j's score counts).
  float pend_v[kQueriesPerWave] = {};
  uint32_t pend_ok = 0;
  auto count_pending = [&](int j) {
    if constexpr (kCount) {
      const uint32_t inc = ((pend_ok >> j) & 1u) << digit_half_shift(pend_v[j]);
      atomicAdd(&bins[(kQueriesPerWave * wave + j) * (kDigitBins / 2) + digit_word(pend_v[j])], inc);
    }
  };
  for (int s = 0; s < stages; ++s) {
    // Wave 0's loads of stage s have landed; stage s - 1 is free.
    if (wave == 0) wait_dma<(kKLoads + kSLoads) * (kRing - 2)>();
    lds_barrier();
    if (wave == 0) {
      issue(s + kRing - 1);
    } else if (s > 0 && wave == 1 + (s - 1) % (kWaves - 1)) {
      store_staged(s - 1);
    }

    const uint32_t stage = ring_base + (uint32_t)(s % kRing) * kStageBytes;
    // The stage's keys in two passes of 64 (lane l of a pass ends with key l).
#pragma unroll
    for (int hf = 0; hf < kStageKeys / kHalfKeys; ++hf) {
      const int64_t key0 = kb + (int64_t)s * kStageKeys + kHalfKeys * hf;
      const uint32_t half = stage + (uint32_t)(kHalfKeys * hf * kDim);

      // B operand of key group u: key 16u + col of the pass, logical chunks 2g,
      // 2g + 1 (the swizzle by key & 7 is the same within the stage).
      auto load_b = [&](int u) -> v8i {
        const int key = 16 * u + col;
        const uint32_t base = half + key * kDim;
        const v4u lo = lds_v4u(base + (((2 * group) ^ (key & 7)) << 4));
        const v4u hi = lds_v4u(base + (((2 * group + 1) ^ (key & 7)) << 4));
        return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      };
      // Units i = 2u + j (key group u, query j): the MFMAs of unit i are issued
      // before the epilogue of unit i - 1.
      constexpr int kUnits = 4 * kQueriesPerWave;
      float part[kQueriesPerWave][4];
      v8i b[2];
      b[0] = load_b(0);
      b[1] = load_b(1);
      v4f acc[2][4];
      v4f acc_lin[2];  // linear half of key group u (parity u & 1), both queries
      auto mfmas = [&](int i) {
        const int u = i / kQueriesPerWave, j = i % kQueriesPerWave;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[i & 1][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              qa[j][t], b[u & 1], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
        if (j == 0)
          acc_lin[u & 1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              qd, b[u & 1], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
      };
      auto epilogue = [&](int i) {
        const int u = i / kQueriesPerWave, j = i % kQueriesPerWave;
        // relu(s) w = (|s| + s) w / 2: the |s| half here, one FMA per head
        // (wt holds w / 2) in one chain over the head tiles in order; the s
        // half is the linear MFMA's share of this lane. (One chain: a wave's
        // dependent FMAs issue back to back, and partial chains would cost
        // three adds per unit.)
        float p = fabsf(acc[i & 1][0][0]) * wt[j][0];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = (t == 0 ? 1 : 0); r < 4; ++r) p = fmaf(fabsf(acc[i & 1][t][r]), wt[j][4 * t + r], p);
        p = fmaf(acc_lin[u & 1][j], fl[j], p);
        // Pins the epilogue here: otherwise instruction selection sinks it below
        // every MFMA of the stage and all 64 results stay live.
        asm volatile("" : "+v"(p));
        part[j][u] = p;
      };
      // The wave's priority falls as it moves through the stage (3 and 2 in
      // the first pass, 1 and 0 in the second). Of the two waves on a SIMD the
      // one behind then wins the issue arbitration, and both reach the
      // barrier at about the same time; by age alone the older wave runs
      // ahead and the younger one finishes the stage with the SIMD to itself.
      if (hf == 0) __builtin_amdgcn_s_setprio(3); else __builtin_amdgcn_s_setprio(1);
      mfmas(0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 1; i < kUnits; ++i) {
        if (i == kUnits / 2) {
          if (hf == 0) __builtin_amdgcn_s_setprio(2); else __builtin_amdgcn_s_setprio(0);
        }
        mfmas(i);
        // b[u & 1] is free once the last query of group u has its MFMAs issued.
        const bool refill = i % kQueriesPerWave == kQueriesPerWave - 1 && i / kQueriesPerWave + 2 < 4;
        if (refill) b[(i / kQueriesPerWave) & 1] = load_b(i / kQueriesPerWave + 2);
        epilogue(i - 1);
        if (i <= kQueriesPerWave) count_pending(i - 1);
        // One MFMA, then the FMAs of one accumulator of the previous unit,
        // four times (five MFMAs with a key group's linear one): the results
        // read were issued a full unit earlier, and the VALU work runs under
        // the MFMAs.
        if (refill) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if (i % kQueriesPerWave == 0) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      epilogue(kUnits - 1);

      const int32_t key = (int32_t)(key0 + lane);
      const bool full = key0 + kHalfKeys <= ke;  // no lane past the split's end
      const float ks = *(const float __attribute__((address_space(3)))*)(uintptr_t)(
          stage + kKBytes + 4 * (kHalfKeys * hf + lane));
#pragma unroll
      for (int j = 0; j < kQueriesPerWave; ++j) {
        const float total = reduce_scatter4(part[j]);
        const bool visible = key >= qs[j] && key < qe[j];
        const float v = visible ? total * ks : neg_inf;
        if constexpr (kCount) {
          pend_v[j] = v;
          pend_ok = (pend_ok & ~(1u << j)) | ((qw + j < rows && key < count_end) ? 1u << j : 0u);
        }
        if (wave == 0) {
          staged[s & 1][j][kHalfKeys * hf + lane] = v;
        } else if (qw + j < rows && (full || key < ke)) {
          out[(qw + j) * ldo + key] = v;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kQueriesPerWave; ++j) count_pending(j);
  if (stages > 0) {
    lds_barrier();  // wave 0's last rows are staged
    if (wave == 1 + (stages - 1) % (kWaves - 1)) store_staged(stages - 1);
  }
  // Drain the DMA issued past the last stage before exit.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Columns of this split at or beyond every causal end: -inf.
  const int64_t tail = kb + (int64_t)stages * kStageKeys;
  if (tail < ke) {
    for (int i = wave; i < kQueriesPerBlock; i += kWaves) {
      const int64_t qi = q0 + i;
      if (qi >= rows) continue;
      for (int64_t key = tail + lane; key < ke; key += 64) out[qi * ldo + key] = neg_inf;
    }
  }
  if constexpr (kCount) {
    __syncthreads();  // the zeroing above, also with no stages
    if (tail < count_end && tid < kQueriesPerBlock && q0 + tid < rows)
      atomicAdd(&bins[tid * (kDigitBins / 2) + (kNegInfDigit & 1023)],
                (uint32_t)(count_end - tail) << ((kNegInfDigit >> 10) << 4));
    __syncthreads();
    // Every word read at once; each nonzero half adds its count to the
    // global counts of its digit.
    v4u words[kBinVecs];
#pragma unroll
    for (int i = 0; i < kBinVecs; ++i) words[i] = reinterpret_cast<const v4u*>(bins)[i * kThreads + tid];
#pragma unroll
    for (int i = 0; i < kBinVecs; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t c = words[i][e];
        if (c == 0) continue;
        const int w = 4 * (i * kThreads + tid) + e;
        uint32_t* dst = digit_counts + (q0 + w / (kDigitBins / 2)) * kDigitBins + w % (kDigitBins / 2);
        if (c & 0xFFFFu) atomicAdd(dst, c & 0xFFFFu);
        if (c >> 16) atomicAdd(dst + kDigitBins / 2, c >> 16);
      }
    }
  }
}

}  // namespace
}  // namespace dsa

namespace dsa {
namespace {

int logits_launch(const void* q, const void* k, const float* weights, const float* kscale,
                  const int32_t* starts, const int32_t* ends, int64_t query_start, int64_t rows,
                  int64_t columns, int64_t ldo, const float* q_fold, float* out,
                  uint32_t* digit_counts, hipStream_t stream) {
  DSA_CHECK_ARG(rows >= 0 && columns >= 1, "logits requires nonempty K");
  DSA_CHECK_ARG(ldo >= columns, "output row stride must cover every column");
  DSA_CHECK_ARG(query_start >= 0 && query_start + rows <= columns,
                "query_start must place all query rows inside the visible KV sequence");
  DSA_CHECK_ARG((starts == nullptr) == (ends == nullptr), "starts and ends go together");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(q && k && weights && kscale && out, "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(weights) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(kscale) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(q_fold) % 16 == 0,
                "q, k, weights and q_fold must be 16-byte aligned");
  DSA_CHECK_ARG(columns * kDim < 0xFFFFFFFFll, "K must be addressable with 32-bit offsets");
  const int64_t qgroups = (rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const int64_t cus = device_cu_count();
  int64_t splits = (cus + qgroups - 1) / qgroups;
  if (splits < 1) splits = 1;
  int64_t per = (ldo + splits - 1) / splits;
  per = (per + kStageKeys - 1) / kStageKeys * kStageKeys;
  if (digit_counts && per > kMaxSplitKeys) per = kMaxSplitKeys;  // 16-bit LDS counters
  splits = (ldo + per - 1) / per;
  // Work-groups are dealt to the eight XCDs round-robin by linear id
  // (x + splits * y): with a multiple of 8 splits every query group of one
  // key range runs on the same XCD and the eight share its keys through that
  // XCD's L2. The added splits start past the last column and exit at once.
  if (splits >= 8) splits = (splits + 7) / 8 * 8;
  DSA_CHECK_ARG(qgroups < 65536, "too many query rows for one launch");
  DSA_CHECK_ARG(ldo < 0x7FFFFFFF - 64, "the logits row stride must fit int32");
  hipLaunchKernelGGL(digit_counts ? logits_fp8_mfma<true> : logits_fp8_mfma<false>,
                     dim3((unsigned)splits, (unsigned)qgroups), dim3(kThreads), 0, stream,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k), weights,
                     kscale, starts, ends, query_start, rows, columns, ldo, per, q_fold, out,
                     digit_counts);
  DSA_CHECK_LAUNCH("indexer logits");
  return kOk;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_indexer_logits_fp8(const void* q, const void* k, const float* weights,
                                      const float* kscale, const int32_t* starts,
                                      const int32_t* ends, int64_t query_start, int64_t rows,
                                      int64_t columns, int64_t ldo, float* out,
                                      hipStream_t stream) {
  return dsa::logits_launch(q, k, weights, kscale, starts, ends, query_start, rows, columns, ldo,
                            nullptr, out, nullptr, stream);
}

extern "C" int dsa_indexer_logits_fp8_folded(const void* q, const void* k, const float* weights,
                                             const float* kscale, const int32_t* starts,
                                             const int32_t* ends, int64_t query_start,
                                             int64_t rows, int64_t columns, int64_t ldo,
                                             const float* q_fold, float* out,
                                             hipStream_t stream) {
  DSA_CHECK_ARG(rows == 0 || q_fold != nullptr, "null pointer");
  return dsa::logits_launch(q, k, weights, kscale, starts, ends, query_start, rows, columns, ldo,
                            q_fold, out, nullptr, stream);
}

extern "C" int dsa_indexer_logits_fp8_counted(const void* q, const void* k, const float* weights,
                                              const float* kscale, const int32_t* starts,
                                              const int32_t* ends, int64_t query_start,
                                              int64_t rows, int64_t columns, int64_t ldo,
                                              const float* q_fold, float* out,
                                              uint32_t* digit_counts, hipStream_t stream) {
  DSA_CHECK_ARG(rows == 0 || (digit_counts != nullptr &&
                              reinterpret_cast<uintptr_t>(digit_counts) % 4 == 0),
                "digit counts must be a 4-byte aligned device pointer");
  return dsa::logits_launch(q, k, weights, kscale, starts, ends, query_start, rows, columns, ldo,
                            q_fold, out, digit_counts, stream);
}


// Logits with their radix-digit counts, then the exact top-k that starts from
// those counts instead of a histogram pass over the scores (the counts are
// zeroed again by the top-k). The scores are still written in full.
extern "C" int dsa_indexer_topk_fp8(const void* q, const void* k, const float* weights,
                                    const float* kscale, const int32_t* starts,
                                    const int32_t* ends, int64_t query_start, int64_t rows,
                                    int64_t columns, int64_t ldo, const float* q_fold,
                                    float* scores, int64_t topk, float* values,
                                    int32_t* indices, int64_t out_ld, void* workspace,
                                    int64_t workspace_bytes, hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(topk >= 1 && topk <= 2048, "k must be an integer in [1, 2048]");
  DSA_CHECK_ARG(rows >= 0 && columns >= 1, "logits requires nonempty K");
  DSA_CHECK_ARG(out_ld >= (topk < columns ? topk : columns), "output row stride too small");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(values && indices, "null pointer");
  int64_t needed = 0;
  const int status_bytes = dsa_indexer_topk_workspace_bytes(rows, columns, &needed);
  if (status_bytes != kOk) return status_bytes;
  DSA_CHECK_ARG(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 8 == 0 &&
                    workspace_bytes >= needed,
                "indexer top-k workspace too small or misaligned");
  // The workspace starts with the [rows][2048] digit counts.
  const int status = logits_launch(q, k, weights, kscale, starts, ends, query_start, rows, columns,
                                   ldo, q_fold, scores, static_cast<uint32_t*>(workspace), stream);
  if (status != kOk) return status;
  return dsa_topk_radix_digits(scores, rows, columns, ldo, topk, values, indices, out_ld, workspace,
                               workspace_bytes, stream);
}
