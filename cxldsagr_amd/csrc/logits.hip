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
//   l of a 64-key pass: one coalesced 256-byte row store. The arithmetic
//   lives in logits_core.h, shared with the exact row recompute of the
//   candidate top-k.
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
//
// Three output modes of the one kernel: plain scores; scores plus their
// radix-digit counts (the level-0 histogram of the top-k); or candidates
// only (the fused indexer top-k): every score at or above its row's floor
// is written as a composite top-k key into the row's list for the split, and
// the score matrix is not written (see logits_fp8_mfma's kModeEmit notes).
#include "logits_core.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

using namespace logits_core;

constexpr int kWaves = 8;
constexpr int kQueriesPerBlock = kWaves * kQueriesPerWave;
constexpr int kStageKeys = 128;                    // keys per DMA stage and barrier
constexpr int kHalfKeys = 64;                      // keys per compute pass (lane = key)
constexpr int kThreads = kWaves * 64;
constexpr int kRing = 4;
constexpr int kKBytes = kStageKeys * kDim;         // 16 KB of keys per stage
constexpr int kKLoads = kKBytes / (64 * 16);       // DMA instructions for the keys (wave 0)
constexpr int kSLoads = kStageKeys / 64;           // DMA instructions for the key scales
constexpr int kStageBytes = kKBytes + kStageKeys * 4;  // + the stage's key scales
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

enum Mode : int { kModePlain = 0, kModeCount = 1, kModeEmit = 2 };

// Candidate output of kModeEmit. Per (row, split): a list of `cap` composite
// keys (radix(v) << 32 | ~column) and a record {listed, spill}: the keys
// listed, and the first column from which the split's scores of that row
// were stored in full into the score matrix instead (INT32_MAX: none).
struct EmitArgs {
  const uint32_t* floors;  // [rows][2] radix-key floors per row (row_floor); 0: store the row in full
  uint64_t* lists;         // [rows][splits][cap]
  uint32_t* records;       // [rows][splits][2]
  int32_t cap;
  int32_t splits;
};

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

// kModeEmit store of one row's 64 scores of a pass (lane = column key0 +
// lane; wave-uniform state): scores at or above the floor go to the list
// (positions from the ballot, no atomics); once fewer than 64 slots are
// left, or from `spill` on, the scores are stored in full instead.
__device__ __forceinline__ void emit_pass(float v, int32_t key0, int lane, uint32_t floor,
                                          int32_t& listed, int32_t& spill, int32_t cap,
                                          float* __restrict__ out_row,
                                          uint64_t* __restrict__ list) {
  if (key0 < spill && listed + kHalfKeys > cap) spill = key0;
  if (key0 >= spill) {
    out_row[key0 + lane] = v;
    return;
  }
  const uint32_t key = radix_of(v);
  const bool hit = key >= floor;
  const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
  if (hit) {
    const uint32_t pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    list[listed + pos] = ((uint64_t)key << 32) | (uint64_t)(~(uint32_t)(key0 + lane));
  }
  listed += __builtin_popcountll(m);
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

// kModeEmit: rows whose floor is 0 are stored in full (as kModePlain, with
// the -inf tail); the others list only their scores at or above the floor,
// per split into a list of `cap` keys, and switch to full stores (from a
// 64-key pass on, recorded in the split's record) when fewer than 64 slots
// are left. No digit counts, and no score of a listing row is stored before
// its spill point.
template <int kMode>
__global__ __launch_bounds__(kThreads, 1) void logits_fp8_mfma(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ k, const float* __restrict__ w,
    const float* __restrict__ kscale, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ ends, int64_t query_start, int64_t rows, int64_t columns,
    int64_t ldo, int64_t keys_per_split, const float* __restrict__ q_fold, float* __restrict__ out,
    uint32_t* __restrict__ digit_counts, EmitArgs emit) {
  constexpr bool kCount = kMode == kModeCount;
  constexpr bool kEmit = kMode == kModeEmit;
  __shared__ __align__(16) uint8_t ring[kRing][kStageBytes];
  // Packed 16-bit digit counts of the block's rows: digit d of row i is half
  // d >> 10 of word i * kDigitBins / 2 + (d & 1023).
  constexpr int kBinWords = kQueriesPerBlock * kDigitBins / 2;
  constexpr int kBinVecs = kBinWords / (4 * kThreads);  // 16-byte LDS accesses per thread
  __shared__ __align__(16) uint32_t bins[kCount ? kBinWords : 4];
  // kModeEmit: wave 0's rows' {listed, spill}, kept by the waves that store
  // those rows in turn.
  __shared__ int32_t w0_state[kQueriesPerWave][2];

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
  // Stage 0's keys are on their way while the query operands load (wave 0's
  // loads complete in issue order, the DMA first); the next stages follow
  // once those have landed, so that their 2 x 17 KB per work-group do not
  // queue ahead of the query operands the first MFMAs wait for (layer
  // -0.35 us against issuing all kRing - 1 stages here).
  if (wave == 0) issue(0);


  // Per-wave query operands and head weights (lane rows: heads 16t + 4g + r).
  // Key positions fit int32 (the launcher checks ldo < 2^31).
  v8i qa[kQueriesPerWave][4];
  float wt[kQueriesPerWave][16];
  int32_t qs[kQueriesPerWave], qe[kQueriesPerWave];
  const int64_t qw = q0 + wave * kQueriesPerWave;

  // Linear half of the head sum (query_digits): q' from four partial sums
  // over heads 16g .. 16g + 15 - from the layer prologue (q_fold,
  // [rows][4][128]) or formed here the same way (fold_partials).
  //
  // Load order: the inputs of q' and the head weights first, then the query
  // operands (the bulk of the bytes), so that forming q' waits only for its
  // own inputs and overlaps the latency of the query operands.
  __shared__ __align__(16) uint8_t digits[kWaves][kQueriesPerWave][kDigits][kDim];
  v8i qd;
  float fl[kQueriesPerWave];
  const int fj = lane >> 5;
  const int fc = lane & 31;
  const bool flive = qw + fj < rows;
  const int64_t fqc = flive ? qw + fj : 0;
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
  // kModeEmit: the floors of this wave's rows and of wave 0's (stored by
  // the other waves), and the list state of this wave's rows.
  uint32_t floor_own[kQueriesPerWave] = {}, floor_w0[kQueriesPerWave] = {};
  int32_t listed[kQueriesPerWave] = {}, spill[kQueriesPerWave] = {};
  if constexpr (kEmit) {
#pragma unroll
    for (int j = 0; j < kQueriesPerWave; ++j) {
      floor_own[j] = qw + j < rows ? row_floor(emit.floors, qw + j) : 0u;
      floor_w0[j] = q0 + j < rows ? row_floor(emit.floors, q0 + j) : 0u;
    }
  }
#pragma unroll
  for (int j = 0; j < kQueriesPerWave; ++j) {
    const int64_t qc = qw + j < rows ? qw + j : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) qa[j][t] = query_operand(q, qc, t, col, group);
  }
  if (!q_fold) fold_partials(codes, w4, flive, pg);
  query_digits(pg, digits[wave], lane, qd, fl);
  if constexpr (kEmit) {
#pragma unroll
    for (int j = 0; j < kQueriesPerWave; ++j) {
      floor_own[j] = __builtin_amdgcn_readfirstlane(floor_own[j]);
      floor_w0[j] = __builtin_amdgcn_readfirstlane(floor_w0[j]);
      // A row without a floor is stored in full from its first column.
      spill[j] = floor_own[j] == 0u ? 0 : 0x7FFFFFFF;
    }
    // Ordered before the first store of wave 0's rows by the first barrier.
    if (wave == 1 && lane < kQueriesPerWave) {
      w0_state[lane][0] = 0;
      w0_state[lane][1] = floor_w0[lane] == 0u ? 0 : 0x7FFFFFFF;
    }
  }
  auto list_of = [&](int64_t row) {
    return emit.lists + (row * emit.splits + blockIdx.x) * (int64_t)emit.cap;
  };

  // Wave 0's finished rows, [stage parity][query][key].
  __shared__ __align__(16) float staged[2][kQueriesPerWave][kStageKeys];
  auto store_staged = [&](int st) {
    if constexpr (kEmit) {
#pragma unroll
      for (int j = 0; j < kQueriesPerWave; ++j) {
        const int64_t qi = q0 + j;  // wave 0's queries
        if (qi >= rows) continue;
        int32_t n = __builtin_amdgcn_readfirstlane(w0_state[j][0]);
        int32_t sp = __builtin_amdgcn_readfirstlane(w0_state[j][1]);
#pragma unroll
        for (int hf = 0; hf < kStageKeys / kHalfKeys; ++hf) {
          const int32_t key0 = (int32_t)(kb + (int64_t)st * kStageKeys + kHalfKeys * hf);
          emit_pass(staged[st & 1][j][kHalfKeys * hf + lane], key0, lane, floor_w0[j], n, sp,
                    emit.cap, out + qi * ldo, list_of(qi));
        }
        if (lane == 0) {
          w0_state[j][0] = n;
          w0_state[j][1] = sp;
        }
      }
    } else {
#pragma unroll
      for (int hf = 0; hf < kStageKeys / kHalfKeys; ++hf) {
        const int64_t key = kb + (int64_t)st * kStageKeys + kHalfKeys * hf + lane;
#pragma unroll
        for (int j = 0; j < kQueriesPerWave; ++j) {
          const int64_t qi = q0 + j;  // wave 0's queries
          if (qi < rows && key < ke) out[qi * ldo + key] = staged[st & 1][j][kHalfKeys * hf + lane];
        }
      }
    }
  };

  // All compiler-visible global loads (and stage 0's DMA) complete here: from
  // now on wave 0's vmcnt counts DMA only. Stages 1 .. kRing - 2 go out now.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  if (wave == 0) {
#pragma unroll
    for (int s = 1; s < kRing - 1; ++s) issue(s);
  }

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
        // relu(s) w = (|s| + s) w / 2 (head_sum). One chain: a wave's
        // dependent FMAs issue back to back, and partial chains would cost
        // three adds per unit.
        float p = head_sum(acc[i & 1], acc_lin[u & 1][j], wt[j], fl[j]);
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
        } else if constexpr (kEmit) {
          // (Stages never reach past the split: its length is a multiple of
          // the stage, and ldo of 256.)
          if (qw + j < rows)
            emit_pass(v, (int32_t)key0, lane, floor_own[j], listed[j], spill[j], emit.cap,
                      out + (qw + j) * ldo, list_of(qw + j));
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

  // Columns of this split at or beyond every causal end: -inf (kModeEmit:
  // only rows stored in full).
  const int64_t tail = kb + (int64_t)stages * kStageKeys;
  if (tail < ke) {
    for (int i = wave; i < kQueriesPerBlock; i += kWaves) {
      const int64_t qi = q0 + i;
      if (qi >= rows) continue;
      if constexpr (kEmit) {
        if (row_floor(emit.floors, qi) != 0u) continue;
      }
      for (int64_t key = tail + lane; key < ke; key += 64) out[qi * ldo + key] = neg_inf;
    }
  }
  if constexpr (kEmit) {
    // Records: waves 1-7 their own rows; wave 0's rows by the wave that
    // stored its last stage (wave 1 without stages).
    const int w0_writer = stages > 0 ? 1 + (stages - 1) % (kWaves - 1) : 1;
    if (wave != 0 && lane < kQueriesPerWave) {
      const int64_t row = qw + lane;
      if (row < rows) {
        uint32_t* rec = emit.records + (row * emit.splits + blockIdx.x) * 2;
        rec[0] = (uint32_t)(lane == 0 ? listed[0] : listed[1]);
        rec[1] = (uint32_t)(lane == 0 ? spill[0] : spill[1]);
      }
    }
    if (wave == w0_writer && lane < kQueriesPerWave && q0 + lane < rows) {
      uint32_t* rec = emit.records + ((q0 + lane) * emit.splits + blockIdx.x) * 2;
      rec[0] = (uint32_t)w0_state[lane][0];
      rec[1] = (uint32_t)w0_state[lane][1];
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

// ---- per-row floors of the candidate top-k (floor_rank, floor_of_samples in
// logits_core.h): one work-group per row scores the row's sample columns
// from the quantised queries and folded weights the logits kernel takes.
constexpr int kFloorThreads = 512;
constexpr int kFloorWaves = kFloorThreads / 64;
constexpr int kFloorBatch = 8;  // 16-sample groups per wave whose loads are in flight together

__global__ __launch_bounds__(kFloorThreads) void index_floors(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ k, const float* __restrict__ w,
    const float* __restrict__ kscale, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ ends, int64_t query_start, int64_t columns, int count,
    uint32_t* __restrict__ floors) {
  __shared__ uint32_t keys[kFloorMaxSamples];
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t wave_sums[kFloorWaves];
  __shared__ uint32_t result[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int group = lane >> 4;
  const int col = lane & 15;
  const int64_t s = starts ? (int64_t)starts[row] : 0;
  int64_t e = ends ? (int64_t)ends[row] : query_start + row + 1;
  if (e > columns) e = columns;
  const int64_t visible = e > s ? e - s : 0;
  if (visible < kFloorMinVisible) {
    if (tid < 2) floors[2 * row + tid] = 0u;
    return;
  }
  const int64_t n = floor_samples(visible, kFloorMaxSamples);
  const int64_t stride = visible / n;  // >= 2
  const uint32_t rank = floor_rank(n, count, visible);
  if (rank > (uint32_t)n) {
    if (tid < 2) floors[2 * row + tid] = 0u;
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) hist[4 * tid + j] = 0;
  if (tid < 4) result[tid] = 0;
  // Sample m is column s + m stride + stride / 2. Wave w scores the 16-sample
  // groups w, w + waves, ... in batches of kFloorBatch whose key loads are
  // issued together: four MFMAs (16 heads each) per group, then
  // sum_h w_h max(s_h, 0) per lane and over the four lane rows.
  const int groups = (int)(n / 16);
  auto sample_key = [&](int g) { return s + (int64_t)(16 * g + col) * stride + stride / 2; };
  v8i qa[4];
  float wv[16];
  for (int g0 = wave; g0 < groups; g0 += kFloorBatch * kFloorWaves) {
    v8i b[kFloorBatch];
    float ks[kFloorBatch];
#pragma unroll
    for (int i = 0; i < kFloorBatch; ++i) {
      const int g = g0 + i * kFloorWaves;
      const int64_t key = sample_key(g < groups ? g : 0);
      b[i] = key_operand(k, key, group);
      ks[i] = kscale[key];
    }
    if (g0 == wave) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        qa[t] = query_operand(q, row, t, col, group);
        const v4f x = *reinterpret_cast<const v4f*>(w + row * kHeads + 16 * t + 4 * group);
#pragma unroll
        for (int r = 0; r < 4; ++r) wv[4 * t + r] = x[r];
      }
    }
#pragma unroll
    for (int i = 0; i < kFloorBatch; ++i) {
      const int g = g0 + i * kFloorWaves;
      float p = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v4f acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            qa[t], b[i], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) p = fmaf(wv[4 * t + r], fmaxf(acc[r], 0.0f), p);
      }
      p += __shfl_xor(p, 16);
      p += __shfl_xor(p, 32);
      if (group == 0 && g < groups) keys[16 * g + col] = radix_of(p * ks[i]);
    }
  }
  __syncthreads();
  const uint32_t floor = floor_of_samples<kFloorThreads>(keys, (int)n, rank, hist, wave_sums, result);
  if (tid < 2) floors[2 * row + tid] = floor;  // one estimate, kept twice
}

}  // namespace
}  // namespace dsa

namespace dsa {
namespace {

// Key range per work-group: the grid is about one work-group per CU.
struct SplitPlan {
  int64_t qgroups, splits, per;
};

SplitPlan split_plan(int64_t rows, int64_t ldo, bool counted) {
  SplitPlan p;
  p.qgroups = (rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const int64_t cus = device_cu_count();
  int64_t splits = (cus + p.qgroups - 1) / p.qgroups;
  if (splits < 1) splits = 1;
  int64_t per = (ldo + splits - 1) / splits;
  per = (per + kStageKeys - 1) / kStageKeys * kStageKeys;
  if (counted && per > kMaxSplitKeys) per = kMaxSplitKeys;  // 16-bit LDS counters
  splits = (ldo + per - 1) / per;
  // Work-groups are dealt to the eight XCDs round-robin by linear id
  // (x + splits * y): with a multiple of 8 splits every query group of one
  // key range runs on the same XCD and the eight share its keys through that
  // XCD's L2. The added splits start past the last column and exit at once.
  if (splits >= 8) splits = (splits + 7) / 8 * 8;
  p.splits = splits;
  p.per = per;
  return p;
}

int check_logits_args(const void* q, const void* k, const float* weights, const float* kscale,
                      const int32_t* starts, const int32_t* ends, int64_t query_start,
                      int64_t rows, int64_t columns, int64_t ldo, const float* q_fold) {
  DSA_CHECK_ARG(rows >= 0 && columns >= 1, "logits requires nonempty K");
  DSA_CHECK_ARG(ldo >= columns, "output row stride must cover every column");
  DSA_CHECK_ARG(query_start >= 0 && query_start + rows <= columns,
                "query_start must place all query rows inside the visible KV sequence");
  DSA_CHECK_ARG((starts == nullptr) == (ends == nullptr), "starts and ends go together");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(q && k && weights && kscale, "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(weights) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(kscale) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(q_fold) % 16 == 0,
                "q, k, weights and q_fold must be 16-byte aligned");
  DSA_CHECK_ARG(columns * kDim < 0xFFFFFFFFll, "K must be addressable with 32-bit offsets");
  DSA_CHECK_ARG(ldo < 0x7FFFFFFF - 64, "the logits row stride must fit int32");
  DSA_CHECK_ARG((rows + kQueriesPerBlock - 1) / kQueriesPerBlock < 65536,
                "too many query rows for one launch");
  return kOk;
}

int logits_launch(const void* q, const void* k, const float* weights, const float* kscale,
                  const int32_t* starts, const int32_t* ends, int64_t query_start, int64_t rows,
                  int64_t columns, int64_t ldo, const float* q_fold, float* out,
                  uint32_t* digit_counts, hipStream_t stream) {
  const int status = check_logits_args(q, k, weights, kscale, starts, ends, query_start, rows,
                                       columns, ldo, q_fold);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(out != nullptr, "null pointer");
  const SplitPlan p = split_plan(rows, ldo, digit_counts != nullptr);
  hipLaunchKernelGGL(digit_counts ? logits_fp8_mfma<kModeCount> : logits_fp8_mfma<kModePlain>,
                     dim3((unsigned)p.splits, (unsigned)p.qgroups), dim3(kThreads), 0, stream,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k), weights,
                     kscale, starts, ends, query_start, rows, columns, ldo, p.per, q_fold, out,
                     digit_counts, EmitArgs{});
  DSA_CHECK_LAUNCH("indexer logits");
  return kOk;
}

// Workspace of the candidate top-k (256-byte aligned parts): floors u32
// [rows][2], records u32 [rows][splits][2], lists u64 [rows][splits][cap].
struct EmitLayout {
  SplitPlan plan;
  int64_t cap;
  int64_t records_offset, lists_offset, bytes;
};

constexpr int64_t kMaxEmitSplits = 512;

int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }

EmitLayout emit_layout(int64_t rows, int64_t columns, int64_t list_cap) {
  EmitLayout l;
  const int64_t ldo = (columns + 255) / 256 * 256;
  l.plan = split_plan(rows, ldo, false);
  // Default: an eighth of the split (~2x the expected candidates of a split
  // at a uniform spread).
  int64_t cap = list_cap > 0 ? list_cap : l.plan.per / 8;
  cap = (cap + 63) / 64 * 64;
  if (cap < 64) cap = 64;
  l.cap = cap;
  l.records_offset = round256(rows * 8);
  l.lists_offset = l.records_offset + round256(rows * l.plan.splits * 8);
  l.bytes = l.lists_offset + rows * l.plan.splits * cap * 8;
  return l;
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

// ---- the fused indexer top-k that writes only candidates.

extern "C" int dsa_indexer_select_workspace_bytes(int64_t rows, int64_t columns, int64_t list_cap,
                                                  int64_t* bytes) {
  using namespace dsa;
  DSA_CHECK_ARG(rows >= 0 && rows < 0x7FFFFFFF && columns >= 1 && columns < 0x7FFFFFFF - 256 &&
                    list_cap >= 0 && bytes != nullptr,
                "invalid indexer select workspace query");
  *bytes = emit_layout(rows, columns, list_cap).bytes;
  return kOk;
}

extern "C" int dsa_indexer_floors_fp8(const void* q, const void* k, const float* weights,
                                      const float* kscale, const int32_t* starts,
                                      const int32_t* ends, int64_t query_start, int64_t rows,
                                      int64_t columns, int64_t topk, uint32_t* floors,
                                      hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(topk >= 1 && topk <= 2048, "k must be an integer in [1, 2048]");
  const int status = check_logits_args(q, k, weights, kscale, starts, ends, query_start, rows,
                                       columns, columns, nullptr);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(floors != nullptr && reinterpret_cast<uintptr_t>(floors) % 4 == 0, "null pointer");
  DSA_CHECK_ARG(rows < 0x7FFFFFFF, "too many rows");
  const int count = (int)(topk < columns ? topk : columns);
  hipLaunchKernelGGL(index_floors, dim3((unsigned)rows), dim3(kFloorThreads), 0, stream,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k), weights,
                     kscale, starts, ends, query_start, columns, count, floors);
  DSA_CHECK_LAUNCH("indexer floors");
  return kOk;
}

extern "C" int dsa_indexer_logits_fp8_emit(const void* q, const void* k, const float* weights,
                                           const float* kscale, const int32_t* starts,
                                           const int32_t* ends, int64_t query_start, int64_t rows,
                                           int64_t columns, int64_t ldo, const float* q_fold,
                                           float* scores, int64_t list_cap, void* workspace,
                                           int64_t workspace_bytes, hipStream_t stream) {
  using namespace dsa;
  const int status = check_logits_args(q, k, weights, kscale, starts, ends, query_start, rows,
                                       columns, ldo, q_fold);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(ldo == (columns + 255) / 256 * 256, "the score stride must be columns rounded up to 256");
  DSA_CHECK_ARG(scores != nullptr, "null pointer");
  const EmitLayout l = emit_layout(rows, columns, list_cap);
  DSA_CHECK_ARG(l.plan.splits <= kMaxEmitSplits, "too many key splits");
  DSA_CHECK_ARG(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 &&
                    workspace_bytes >= l.bytes,
                "indexer select workspace too small or misaligned");
  uint8_t* base = static_cast<uint8_t*>(workspace);
  EmitArgs emit{reinterpret_cast<const uint32_t*>(base),
                reinterpret_cast<uint64_t*>(base + l.lists_offset),
                reinterpret_cast<uint32_t*>(base + l.records_offset), (int32_t)l.cap,
                (int32_t)l.plan.splits};
  hipLaunchKernelGGL(logits_fp8_mfma<kModeEmit>, dim3((unsigned)l.plan.splits, (unsigned)l.plan.qgroups),
                     dim3(kThreads), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(k), weights, kscale, starts, ends, query_start,
                     rows, columns, ldo, l.plan.per, q_fold, scores, nullptr, emit);
  DSA_CHECK_LAUNCH("indexer logits (candidates)");
  return kOk;
}

extern "C" int dsa_indexer_emit_topk(const void* q, const void* k, const float* weights,
                                     const float* kscale, const int32_t* starts,
                                     const int32_t* ends, int64_t query_start, int64_t rows,
                                     int64_t columns, const float* q_fold, float* scores,
                                     int64_t topk, float* values, int32_t* indices,
                                     int64_t out_ld, int64_t list_cap, const void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(topk >= 1 && topk <= 2048, "k must be an integer in [1, 2048]");
  const int status = check_logits_args(q, k, weights, kscale, starts, ends, query_start, rows,
                                       columns, columns, q_fold);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(out_ld >= (topk < columns ? topk : columns), "output row stride too small");
  DSA_CHECK_ARG(values && indices && scores, "null pointer");
  const EmitLayout l = emit_layout(rows, columns, list_cap);
  DSA_CHECK_ARG(l.plan.splits <= kMaxEmitSplits, "too many key splits");
  DSA_CHECK_ARG(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 &&
                    workspace_bytes >= l.bytes,
                "indexer select workspace too small or misaligned");
  const uint8_t* base = static_cast<const uint8_t*>(workspace);
  return topk_from_candidates(
      static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k), weights, kscale, starts,
      ends, query_start, q_fold, scores, rows, columns, (columns + 255) / 256 * 256, topk, values,
      indices, out_ld, reinterpret_cast<const uint32_t*>(base),
      reinterpret_cast<const uint32_t*>(base + l.records_offset),
      reinterpret_cast<const uint64_t*>(base + l.lists_offset), l.plan.splits, l.plan.per, l.cap,
      stream);
}

// Floors, candidate logits and the top-k from the candidates, in one call.
extern "C" int dsa_indexer_select_fp8(const void* q, const void* k, const float* weights,
                                      const float* kscale, const int32_t* starts,
                                      const int32_t* ends, int64_t query_start, int64_t rows,
                                      int64_t columns, const float* q_fold, float* scores,
                                      int64_t topk, float* values, int32_t* indices,
                                      int64_t out_ld, void* workspace, int64_t workspace_bytes,
                                      hipStream_t stream) {
  using namespace dsa;
  int status = dsa_indexer_floors_fp8(q, k, weights, kscale, starts, ends, query_start, rows,
                                      columns, topk, static_cast<uint32_t*>(workspace), stream);
  if (status != kOk || rows == 0) return status;
  const int64_t ldo = (columns + 255) / 256 * 256;
  status = dsa_indexer_logits_fp8_emit(q, k, weights, kscale, starts, ends, query_start, rows,
                                       columns, ldo, q_fold, scores, 0, workspace, workspace_bytes,
                                       stream);
  if (status != kOk) return status;
  return dsa_indexer_emit_topk(q, k, weights, kscale, starts, ends, query_start, rows, columns,
                               q_fold, scores, topk, values, indices, out_ld, 0, workspace,
                               workspace_bytes, stream);
}
