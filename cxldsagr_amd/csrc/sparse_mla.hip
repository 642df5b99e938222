// A7/A8: sparse MLA prefill over selected token records, bf16 MFMA with an
// online softmax, from either flat bf16 records (576 x bf16 = 1152 B/token)
// or the fp8 paged cache (656 B/token: 512 e4m3 + 4 fp32 tile scales + 64
// bf16 RoPE, 64 tokens per page).
//
// Semantics: operators/deepseek_v32/attention/reference/torch.py:13-28 - per
// query row r, every selected id in [0, N) (duplicates count per slot) gives
// a record; P = softmax(q[r,h] . rec * scale); out[r,h] = P @ rec[:512],
// rounded to bf16; a row with no valid id is zero.
//
// Mapping (gfx950, wave64). A work-group owns one query row and 64 heads
// and walks the selection in blocks of 32 keys with 4 waves, one per SIMD,
// in two roles, so that the matrix work of one role runs beside the
// conversion and LDS stores of the other (MFMA and VALU work of one wave
// serialise on its SIMD):
// * Score waves 0 and 1 compute S^T = K Q^T for all 32 keys and heads
//   32 sw .. 32 sw + 31 with v_mfma_f32_32x32x16_bf16 (Q^T of their 32 heads
//   stays in AGPRs, 144 registers), then the online softmax of their heads,
//   writing P^T (bf16) and the per-head rescale factors to LDS.
// * Load waves 2 and 3 stage the records: lane (kk, j) (kk = 16 (w - 2) +
//   lane / 4, j = lane % 4) loads a quarter of key kk's record with 16-byte
//   loads, kLookahead blocks ahead, and converts it into bf16 rows of one of
//   three LDS buffers the step before the block is scored (fp8 records by
//   v_cvt_scalef32_pk_bf16_fp8 with their tile scales; e4m3 x 2^k is exact in
//   bf16). Conversion happens once per key, not once per wave that reads it.
// * After the block's barrier all four waves accumulate O^T += V^T P^T
//   (v_mfma_f32_16x16x32_bf16) over all 64 heads: score waves for 48 dims
//   each, load waves for 208 each, which evens out the two roles' time per
//   block. V^T comes from ds_read_b64_tr_b16: lane 4 jj + qq of row group g
//   addresses key 2 jj + 8 (g & 1) + (g >> 1) (and + 16) at dims d0 + 4 qq.
// * Row sums come out of the same MFMA pipe: wave w adds P^T of head tile w
//   against a row of ones, so l sums exactly the bf16 P the product used.
// A buffer written in step b - 1 is read by the scores of block b and,
// after that block's barrier, by its PV product, hence three buffers; P and
// the rescale factors are double buffered by block parity.
//
// Online softmax in log2 units with lazy rescaling (only when a block raises
// a head's running max by more than 8, so p <= 2^8).
#include <type_traits>

#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));

constexpr int kQkDim = 576;
constexpr int kVDim = 512;
constexpr int kHeadsPerGroup = 64;
constexpr int kBlock = 32;            // keys per block
constexpr int kThreads = 256;
constexpr int kMaxSelected = 4096;    // rows table capacity per query row
constexpr int kPageTokens = 64;
constexpr float kRescaleThreshold = 8.0f;

template <bool kFp8>
struct Format {
  static constexpr int kRecordBytes = kFp8 ? 656 : kQkDim * 2;
  // 16-byte loads per lane per block: the two load waves fetch 16 keys each,
  // four lanes per key (fp8: 8 latent + scales + 2 RoPE; bf16: 16 + 2).
  static constexpr int kLoads = kFp8 ? 11 : 18;
};

// bf16 K/V rows of one block in LDS: key r at kRowBytes r, its 576 dims in
// order. 1168 bytes = 292 dwords = 36 (mod 64): the 16 keys read by a 16-lane
// group of the score operands land on 16 distinct 4-bank groups, and the 8
// even (or odd) keys of a V^T transpose read on disjoint 8-bank windows.
constexpr int kRowBytes = kQkDim * 2 + 16;
constexpr int kBufBytes = kBlock * kRowBytes;
constexpr int kBuffers = 3;
// 16-dim tiles of O^T per score wave and per load wave (two of each).
constexpr int kScoreDimTiles = 3;
constexpr int kLoadDimTiles = (kVDim / 16 - 2 * kScoreDimTiles) / 2;

struct __align__(16) Lds {
  uint8_t kv[kBuffers][kBufBytes];
  // P^T in PV B-operand order, by block parity: [parity][head tile][lane]
  // 16 bytes: lane (c, g) of tile t holds head 16t + c, k-index j = key
  // 2(j & 3) + 8(g & 1) + (g >> 1) + 16(j >> 2), bf16.
  uint8_t p[2][4][64][16];
  float alpha[2][kHeadsPerGroup];  // per-head rescale factor of the block, by parity
  float row_sum[kHeadsPerGroup];
  int32_t rows[kMaxSelected];  // physical record row per selected position, -1 = padding
};

// Key order inside a block. Row m = 8a + 4h + i of the 32x32 score tile holds
// key 2i + 8(a & 1) + h + 16(a >> 1); k-index j of the PV operands of lane
// row-group g is key 2(j & 3) + 8(g & 1) + (g >> 1) + 16(j >> 2). With these,
// the four results a score lane holds in registers 4a'..4a'+3 are exactly
// the four consecutive k-indices 4(a' >> 1) .. +3 of one PV operand slot.
__device__ __forceinline__ int score_key(int m) {
  return 2 * (m & 3) + 8 * ((m >> 3) & 1) + ((m >> 2) & 1) + 16 * (m >> 4);
}

// Source of padding slots and invalid ids: a zero record (zero scales), so
// that their V^T operands are zeros rather than whatever the cache holds.
__device__ __align__(16) uint8_t zero_record[kQkDim * 2];

__device__ __forceinline__ v8bf as_v8bf(v4u v) { return __builtin_bit_cast(v8bf, v); }

// Two floats -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){lo, hi}, v2bf));
}

template <bool kHigh>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t word, float scale) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, scale, kHigh));
}

typedef float v16f __attribute__((ext_vector_type(16)));

// acc += a b with the 32x32x16 bf16 MFMA, b (Q^T) pinned to AGPRs: Q^T of 32
// heads (144 registers) does not fit the VGPRs beside the O accumulators, and
// as a compiler-chosen spill it is copied back into an aligned tuple before
// every use. As inline assembly the MFMA is invisible to the hazard
// recognizer, so it covers its own wait states: the leading s_nop 1 gives the
// 2 required after a VALU write of `a` or `acc`; back-to-back MFMAs into the
// same accumulator need none; the reader of the final accumulator waits with
// mfma_drain32().
__device__ __forceinline__ void mfma32_qb(v16f& acc, v8bf a, v8bf b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "a"(b));
}
// Wait states between the last inline-assembly MFMA and any read of its
// results (more than the 18 a 16-pass XDL op needs). The accumulator is an
// operand, so no read of it can be scheduled above the wait.
__device__ __forceinline__ void mfma_drain32(v16f& a) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a));
}

typedef v4s __attribute__((address_space(3))) * lds_v4s;

template <typename T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
  return *(T __attribute__((address_space(3)))*)(uintptr_t)addr;
}
template <typename T>
__device__ __forceinline__ void lds_store(uint32_t addr, T v) {
  *(T __attribute__((address_space(3)))*)(uintptr_t)addr = v;
}

// LDS barrier: finish this wave's LDS traffic, then s_barrier. The memory
// clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <bool kFp8>
__global__ __launch_bounds__(kThreads, 1) void sparse_mla_fwd(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv,
    const int32_t* __restrict__ page_table, int64_t n_tokens, int64_t pages,
    const int32_t* __restrict__ indices, int64_t heads, int64_t topk, float scale_log2,
    uint16_t* __restrict__ out) {
  using F = Format<kFp8>;
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int64_t row = blockIdx.x;
  const int64_t head0 = (int64_t)blockIdx.y * kHeadsPerGroup;
  const int32_t* ids = indices + row * topk;
  const float neg_inf = -__builtin_inff();
  // Blocks of 32 selected positions, rounded up to an even count (the loop
  // takes two per trip; a padding block has no valid key and adds nothing).
  const int n_blocks = (int)((topk + 2 * kBlock - 1) / (2 * kBlock)) * 2;

  // Physical record row of selected position i; -1 for padding, an id
  // outside [0, n_tokens) or a page outside the cache.
  auto phys_of = [&](int i) -> int32_t {
    int32_t phys = -1;
    if (i < topk) {
      const int64_t id = ids[i];
      if (id >= 0 && id < n_tokens) {
        if (kFp8) {
          const int64_t page = page_table[id / kPageTokens];
          if (page >= 0 && page < pages) phys = (int32_t)(page * kPageTokens + id % kPageTokens);
        } else {
          phys = (int32_t)id;
        }
      }
    }
    return phys;
  };

  // Roles: waves 0 and 1 score (32 heads each, all 32 keys of a block, with
  // 32x32x16 MFMAs) and run the softmax; waves 2 and 3 stage the records of
  // the next block (HBM -> registers -> bf16 rows in LDS). All four then
  // accumulate O^T for their share of the 512 dims over all 64 heads.
  const bool scorer = wave < 2;
  const int sw = wave & 1;           // score wave: heads 32 sw .. + 31
  const int n = lane & 31;           // score lane: head 32 sw + n
  const int h = lane >> 5;           // score lane: row half
  // One register pool serves both roles, so that the allocator can give
  // the two roles the same registers: Q^T operands on score waves (k-step
  // ks: dims 16 ks + 8h), staged record bytes on load waves (fp8: two sets
  // of kLoads at 0 and kLoads, bf16: one set).
  constexpr int kPool = kQkDim / 16;
  static_assert((kFp8 ? 2 : 1) * F::kLoads <= kPool, "staging does not fit the pool");
  v4u pool[kPool];
  if (scorer) {
    const uint16_t* qrow = q + ((row * heads + head0 + 32 * sw + n) * kQkDim) + 8 * h;
#pragma unroll
    for (int ks = 0; ks < kPool; ++ks) pool[ks] = *reinterpret_cast<const v4u*>(qrow + 16 * ks);
  }
  float m_run = neg_inf;  // score lane: running max of its head (scaled)
  // Row sums of heads 16 wave + c (P^T against ones; every row alike).
  v4f l_acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // Load role: key kk of each block, quarter j of its record.
  const int kk = 16 * (wave & 1) + (lane >> 2);
  const int j = lane & 3;
  const uint32_t rows_base = (uint32_t)(uintptr_t)&lds.rows[0];
  const uint32_t kv_base = (uint32_t)(uintptr_t)&lds.kv[0][0];
  const uint32_t p_base = (uint32_t)(uintptr_t)&lds.p[0][0][0][0];

  // Per-block base addresses are formed once and hidden from the optimizer:
  // otherwise it hoists (lane offset + constant) out of the loop and pays an
  // add per LDS access instead of using the instruction's offset field.
  auto lane_base = [](uint32_t buf, uint32_t lane_off) -> uint32_t {
    uint32_t a = buf + lane_off;
    asm volatile("" : "+v"(a));
    return a;
  };
  // Block b's record bytes of this lane -> registers. Blocks past the end
  // (and invalid ids) read the zero record, so the load count per block is
  // fixed. fp8 latent loads i cover record bytes 64i + 16j (64 contiguous
  // bytes per key and instruction); bf16 loads 2i + u cover 128i + 32j + 16u.
  auto row_of = [&](int b) -> int32_t {
    return b < n_blocks ? lds_load<int32_t>(rows_base + 4 * (uint32_t)(b * kBlock + kk)) : -1;
  };
  auto fetch = [&](auto set, int32_t phys) __attribute__((always_inline)) {
    v4u* st = pool + decltype(set)::value;
    const uint8_t* rec = phys >= 0 ? kv + (int64_t)phys * F::kRecordBytes : zero_record;
    if (kFp8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) st[i] = *reinterpret_cast<const v4u*>(rec + 64 * i + 16 * j);
      st[8] = *reinterpret_cast<const v4u*>(rec + kVDim);
      st[9] = *reinterpret_cast<const v4u*>(rec + kVDim + 16 + 32 * j);
      st[10] = *reinterpret_cast<const v4u*>(rec + kVDim + 32 + 32 * j);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        st[i] = *reinterpret_cast<const v4u*>(rec + 128 * (i >> 1) + 32 * j + 16 * (i & 1));
      st[16] = *reinterpret_cast<const v4u*>(rec + 2 * kVDim + 32 * j);
      st[17] = *reinterpret_cast<const v4u*>(rec + 2 * kVDim + 16 + 32 * j);
    }
  };
  // Landed record bytes -> bf16 rows of a block buffer (fp8: e4m3 x tile
  // scale, exact in bf16).
  auto unpack = [&](auto set, uint32_t buf) __attribute__((always_inline)) {
    const v4u* st = pool + decltype(set)::value;
    const uint32_t rec = lane_base(buf, (uint32_t)kk * kRowBytes + 32 * j);
    if (kFp8) {
      const v4f sc = __builtin_bit_cast(v4f, st[8]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float s_i = sc[i >> 1];
        const v4u w = st[i];
        const v4u lo{dequant_pair<false>(w.x, s_i), dequant_pair<true>(w.x, s_i),
                     dequant_pair<false>(w.y, s_i), dequant_pair<true>(w.y, s_i)};
        const v4u hi{dequant_pair<false>(w.z, s_i), dequant_pair<true>(w.z, s_i),
                     dequant_pair<false>(w.w, s_i), dequant_pair<true>(w.w, s_i)};
        lds_store<v4u>(rec + 128 * i, lo);
        lds_store<v4u>(rec + 128 * i + 16, hi);
      }
      lds_store<v4u>(rec + 2 * kVDim, st[9]);
      lds_store<v4u>(rec + 2 * kVDim + 16, st[10]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) lds_store<v4u>(rec + 128 * (i >> 1) + 16 * (i & 1), st[i]);
      lds_store<v4u>(rec + 2 * kVDim, st[16]);
      lds_store<v4u>(rec + 2 * kVDim + 16, st[17]);
    }
  };

  // Score A operand (K): lane l reads key score_key(l % 32), dims 16 ks + 8h.
  const uint32_t k_lane = (uint32_t)score_key(n) * kRowBytes + 16 * h;
  // O^T dims of the wave: score waves take fewer (they also run S and the
  // softmax), so that both roles spend about the same time per block.
  const int dim0 = scorer ? 16 * kScoreDimTiles * sw : 16 * (2 * kScoreDimTiles + kLoadDimTiles * (wave & 1));
  // V^T rows (ds_read_b64_tr_b16): lane 4 jj + qq of row group g addresses
  // key 2 jj + 8 (g & 1) + (g >> 1) (and + 16) at dims dim0 + 16m + 4qq.
  const int jj = c >> 2;
  const int qq = c & 3;
  const int vkey = 2 * jj + 8 * (g & 1) + (g >> 1);
  const uint32_t v_lane = (uint32_t)vkey * kRowBytes + 2 * dim0 + 8 * qq;
  constexpr uint32_t kHalf = 16 * kRowBytes;

  // Record loads run kLookahead blocks ahead of the block being scored: two
  // register sets for fp8 (blocks it + 2 and it + 3 in flight), one for the
  // bf16 record, whose two sets would not fit beside O^T.
  constexpr int kLookahead = kFp8 ? 3 : 2;
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, kFp8 ? F::kLoads : 0>;
  // Prologue: the rows table of all positions, blocks 0 .. kLookahead - 1
  // requested and block 0 converted. In the loop the row of the next block
  // to fetch is read from the table one step ahead.
  for (int i = threadIdx.x; i < n_blocks * kBlock; i += kThreads) lds.rows[i] = phys_of(i);
  __syncthreads();  // rows table
  int32_t phys_next = -1;
  if (!scorer) {
    fetch(Set0{}, row_of(0));
    if (kFp8) fetch(Set1{}, row_of(1));
    unpack(Set0{}, kv_base);
    fetch(Set0{}, row_of(kLookahead - 1));
    phys_next = row_of(kLookahead);
  }
  lds_barrier();

  int buf_cur = 0;  // buffer of block it
  // kScore is the wave's role, a compile-time constant of each of the two
  // loops below: with one loop per role the wait-count pass sees only that
  // role's loads and waits for exactly the set being unpacked.
  // ka: the first kAheadK K operands of block it, read before the step (in
  // the previous step's PV phase: block it + 1's rows are complete once
  // block it's barrier has passed).
  constexpr int kAheadK = 6;
  auto k_prefetch = [&](v4u (&ka)[kAheadK], uint32_t buf) __attribute__((always_inline)) {
    const uint32_t kbase = lane_base(buf, k_lane);
#pragma unroll
    for (int d = 0; d < kAheadK; ++d) ka[d] = lds_load<v4u>(kbase + 32 * d);
  };
  auto step = [&](int it, auto set, auto role, auto& o, v4u (&ka)[kAheadK]) __attribute__((always_inline)) {
    constexpr bool kScore = decltype(role)::value;
    constexpr int kM = kScore ? kScoreDimTiles : kLoadDimTiles;
    const uint32_t buf = kv_base + (uint32_t)buf_cur * kBufBytes;
    const int buf_next_i = buf_cur + 1 == kBuffers ? 0 : buf_cur + 1;
    const uint32_t parity = (uint32_t)(it & 1);

    if constexpr (kScore) {
      // ---- S^T = K Q^T: 32 keys x heads 32 sw .. + 31, 36 k-steps of 16
      // dims accumulated back to back.
      // Valid keys of the block (bit = key), read ahead of the MFMAs.
      const int32_t prow = lds_load<int32_t>(rows_base + 4 * (uint32_t)(it * kBlock + n));
      v16f sa = {};
      const uint32_t kbase = lane_base(buf, k_lane);
#pragma unroll
      for (int ks = 0; ks < kQkDim / 16; ++ks) {
        const v8bf a = as_v8bf(ka[ks % kAheadK]);
        if (ks + kAheadK < kQkDim / 16) ka[ks % kAheadK] = lds_load<v4u>(kbase + 32 * (ks + kAheadK));
        mfma32_qb(sa, a, as_v8bf(pool[ks]));
      }
      const uint32_t vmask = (uint32_t)__builtin_amdgcn_ballot_w64(h == 0 && prow >= 0);
      mfma_drain32(sa);

      // ---- online softmax of head 32 sw + n over the block: this lane holds
      // keys score_key(8(r / 4) + 4h + r % 4), the other half (lane ^ 32)
      // the rest. Maxima are taken on raw scores (scale_log2 > 0) and invalid
      // keys become -inf, so p = exp2(s * scale_log2 - m) is one FMA and one
      // exp2. Row sums are not formed here: the PV product adds P^T against a
      // row of ones (the same bf16 P, so O / l is a weighted mean of V).
      float sc[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = sa[r];
      if (vmask != 0xFFFFFFFFu) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = score_key(8 * (r >> 2) + 4 * h + (r & 3));
          sc[r] = (vmask >> key) & 1u ? sc[r] : neg_inf;
        }
      }
      float mx = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
      for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sc[r]), sc[r + 1]);
      mx = fmaxf(mx, sc[15]);
      {
        const uint32_t u = __float_as_uint(mx);
        const auto sw32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        mx = fmaxf(__uint_as_float(sw32[0]), __uint_as_float(sw32[1])) * scale_log2;
      }
      const bool need = mx > m_run + kRescaleThreshold || (m_run == neg_inf && mx != neg_inf);
      const float m_new = need ? fmaxf(m_run, mx) : m_run;
      // exp2(-inf) = 0 covers the first valid block.
      const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      m_run = m_new;
      // With no valid key so far every score is -inf and p = exp2(-inf) = 0.
      const float neg_m = m_run == neg_inf ? 0.0f : -m_run;
      uint32_t pk[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2)
        pk[r / 2] = pack_bf16(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, neg_m)),
                              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r + 1], scale_log2, neg_m)));
      if (h == 0) lds.alpha[parity][32 * sw + n] = alpha;
      // P^T -> LDS: registers 4a' .. 4a' + 3 are k-indices 4(a' >> 1) .. +3 of
      // operand slot (c = n % 16, g = 2h + (a' & 1)) of head tile 2 sw + n / 16.
      const uint32_t p_tile = p_base + parity * 4096 + (uint32_t)((2 * sw + (n >> 4)) * 64 + (n & 15)) * 16;
#pragma unroll
      for (int ap = 0; ap < 4; ++ap) {
        const int gg = 2 * h + (ap & 1);
        lds_store<v2u>(p_tile + (uint32_t)gg * 256 + 8 * (ap >> 1), v2u{pk[2 * ap], pk[2 * ap + 1]});
      }
    } else {
      // ---- block it + 1 -> bf16 rows (its buffer last held block it - 2,
      // whose readers all passed the previous barrier); block
      // it + kLookahead -> the freed registers.
      unpack(set, kv_base + (uint32_t)buf_next_i * kBufBytes);
      fetch(set, phys_next);
      phys_next = row_of(it + kLookahead + 1);
    }
    // The first V^T operands of this block (its rows are complete since the
    // previous barrier) are read before the barrier.
    const uint32_t vbase = lane_base(buf, v_lane);
    auto v_addr = [&](int m) -> uint32_t { return vbase + 32 * m; };
    constexpr int kAhead = 2;
    v4s vlo[kAhead], vhi[kAhead];
#pragma unroll
    for (int d = 0; d < kAhead; ++d) {
      vlo[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)v_addr(d));
      vhi[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(v_addr(d) + kHalf));
    }
    lds_barrier();  // P, alpha and block it + 1's rows visible

    // ---- O^T += V^T P^T for dims dim0 .. dim0 + 16 kM - 1, all 64 heads.
    // Reads first (rescale factors, P^T, then the score waves' first K
    // operands of block it + 1), then the rescale of O^T if any head's
    // running max rose.
    float al[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) al[t] = lds.alpha[parity][16 * t + c];
    v8bf pb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      pb[t] = as_v8bf(lds_load<v4u>(p_base + parity * 4096 + (uint32_t)(t * 64 + lane) * 16));
    const v8bf p_own = as_v8bf(lds_load<v4u>(p_base + parity * 4096 + (uint32_t)(wave * 64 + lane) * 16));
    if constexpr (kScore) k_prefetch(ka, kv_base + (uint32_t)buf_next_i * kBufBytes);
    bool rescale = false;
#pragma unroll
    for (int t = 0; t < 4; ++t) rescale |= al[t] != 1.0f;
    if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int m = 0; m < kM; ++m) o[t][m] *= al[t];
      l_acc *= lds.alpha[parity][16 * wave + c];
    }
    {
      const v4u ones = v4u{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      l_acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(ones), p_own, l_acc, 0, 0, 0);
    }
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const v8bf a = __builtin_bit_cast(
          v8bf, __builtin_shufflevector(vlo[m % kAhead], vhi[m % kAhead], 0, 1, 2, 3, 4, 5, 6, 7));
      if (m + kAhead < kM) {
        vlo[m % kAhead] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)v_addr(m + kAhead));
        vhi[m % kAhead] =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(v_addr(m + kAhead) + kHalf));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[t], o[t][m], 0, 0, 0);
    }
    buf_cur = buf_next_i;
  };
  // Two blocks per trip so that each register set stays a fixed register set.
  auto run = [&](auto role) __attribute__((always_inline)) {
    constexpr int kM = decltype(role)::value ? kScoreDimTiles : kLoadDimTiles;
    // O^T: head tile t (heads 16t + c), dims dim0 + 16m + 4g + r.
    v4f o[4][kM];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int m = 0; m < kM; ++m) o[t][m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    v4u ka[kAheadK];
    if constexpr (decltype(role)::value) k_prefetch(ka, kv_base);
    for (int it = 0; it < n_blocks; it += 2) {
      step(it, Set1{}, role, o, ka);
      step(it + 1, Set0{}, role, o, ka);
    }
    // The fetches past the last block are never read; let them land before
    // the registers are released.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- row sums of all 64 heads, then O / l.
    if (g == 0) lds.row_sum[16 * wave + c] = l_acc[0];
    __syncthreads();
    uint16_t* obase = out + ((row * heads + head0 + c) * kVDim) + dim0 + 4 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float lt = lds.row_sum[16 * t + c];
      const float inv_l = lt > 0.0f ? 1.0f / lt : 0.0f;
      uint16_t* orow = obase + (int64_t)16 * t * kVDim;
#pragma unroll
      for (int m = 0; m < kM; ++m)
        *reinterpret_cast<uint2*>(orow + 16 * m) =
            make_uint2(pack_bf16(o[t][m][0] * inv_l, o[t][m][1] * inv_l),
                       pack_bf16(o[t][m][2] * inv_l, o[t][m][3] * inv_l));
    }
  };
  if (scorer) run(std::true_type{});
  else run(std::false_type{});
}

template <bool kFp8>
int launch(const void* q, int64_t rows, int64_t heads, const void* kv, const int32_t* page_table,
           int64_t n_tokens, int64_t pages, const int32_t* indices, int64_t topk, float scale,
           void* out, hipStream_t stream) {
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(sparse_mla_fwd<kFp8>, dim3((unsigned)rows, (unsigned)(heads / kHeadsPerGroup)),
                     dim3(kThreads), 0, stream, static_cast<const uint16_t*>(q),
                     static_cast<const uint8_t*>(kv), page_table, n_tokens, pages, indices, heads,
                     topk, scale_log2, static_cast<uint16_t*>(out));
  DSA_CHECK_LAUNCH("sparse MLA");
  return kOk;
}

int check_common(const void* q, int64_t rows, int64_t heads, const int32_t* indices, int64_t topk,
                 float scale, void* out) {
  DSA_CHECK_ARG(rows >= 0 && topk >= 1, "invalid sparse MLA shape");
  DSA_CHECK_ARG(topk <= kMaxSelected, "sparse MLA supports at most 4096 selected tokens per row");
  DSA_CHECK_ARG(heads > 0 && heads % kHeadsPerGroup == 0 && heads / kHeadsPerGroup < 65536,
                "heads must be a positive multiple of 64");
  DSA_CHECK_ARG(__builtin_isfinite(scale), "scale must be finite");
  DSA_CHECK_ARG(rows < 0x7FFFFFFF, "too many query rows");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(q && indices && out, "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0,
                "q must be 16-byte and out 8-byte aligned");
  return kOk;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_sparse_mla_bf16(const void* q, int64_t rows, int64_t heads, const void* kv,
                                   int64_t kv_rows, const int32_t* indices, int64_t topk,
                                   float scale, void* out, hipStream_t stream) {
  using namespace dsa;
  int status = check_common(q, rows, heads, indices, topk, scale, out);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(kv_rows >= 1 && kv_rows < 0x7FFFFFFF, "KV row count must be in [1, 2^31)");
  DSA_CHECK_ARG(kv != nullptr, "null kv");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(kv) % 16 == 0, "kv must be 16-byte aligned");
  return launch<false>(q, rows, heads, kv, nullptr, kv_rows, 0, indices, topk, scale, out,
                       stream);
}

extern "C" int dsa_sparse_mla_fp8_paged(const void* q, int64_t rows, int64_t heads,
                                        const void* cache, int64_t pages,
                                        const int32_t* page_table, int64_t n_tokens,
                                        const int32_t* indices, int64_t topk, float scale,
                                        void* out, hipStream_t stream) {
  using namespace dsa;
  int status = check_common(q, rows, heads, indices, topk, scale, out);
  if (status != kOk || rows == 0) return status;
  DSA_CHECK_ARG(pages >= 1 && n_tokens >= 1 && n_tokens < 0x7FFFFFFF,
                "need a nonempty cache and 1 <= n_tokens < 2^31");
  DSA_CHECK_ARG(pages * kPageTokens < 0x7FFFFFFF, "cache rows must fit int32");
  DSA_CHECK_ARG(cache && page_table, "null cache or page table");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(cache) % 16 == 0, "cache must be 16-byte aligned");
  return launch<true>(q, rows, heads, cache, page_table, n_tokens, pages, indices, topk, scale,
                      out, stream);
}
