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
// in two roles:
// * Score waves 0 and 1 compute S^T = K Q^T for all 32 keys and heads
//   32 sw .. 32 sw + 31 with v_mfma_f32_32x32x16_bf16 (Q^T of their 32 heads
//   stays in 144 AGPRs, read by the MFMAs as the B operand), and the online
//   softmax of their heads, writing P^T (bf16) and per-head rescale factors
//   to LDS.
// * Load waves 2 and 3 stage the records: lane (kk, j) (kk = 16 (w - 2) +
//   lane / 4, j = lane % 4) loads a quarter of key kk's record with 16-byte
//   loads, kLookahead blocks ahead, and converts it into bf16 rows of a
//   block buffer in LDS (fp8 records by v_cvt_scalef32_pk_bf16_fp8 with
//   their tile scales; e4m3 x 2^k is exact in bf16), once per key.
// * All four accumulate O^T += V^T P^T (v_mfma_f32_16x16x32_bf16, V^T from
//   ds_read_b64_tr_b16) over all 64 heads: score waves for 96 dims each,
//   load waves for 160 each. Row sums come from the same MFMA pipe: each
//   wave adds P^T of one head tile against a row of ones, so l sums exactly
//   the bf16 P the product used.
// The work is software-pipelined so that every wave has matrix work and
// independent VALU / LDS work in the same step, which its SIMD runs side by
// side (the code issues them interleaved): in step `it` the score waves
// compute S(it) and the softmax of block it - 1 (its scores kept in
// registers) and the PV product of block it - 2; the load waves convert the
// rows of block it + 1 and run the PV product of block it - 2. One barrier
// per step; four block buffers (S reads it, PV reads it - 2, it + 1 is
// written); P and the rescale factors are double buffered by block parity.
// The physical rows of the selection live in a ring of 8 blocks in LDS that
// the load waves keep 6 blocks ahead (the id and page-table loads each
// land two steps before use, ahead of the record loads).
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
constexpr int kMaxSelected = 4096;    // widest selection per query row
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
constexpr int kBuffers = 4;
// Physical rows of the selected keys, by block, in a ring of kRing blocks
// filled kRingAhead blocks ahead of the block being scored.
constexpr int kRing = 8;
constexpr int kRingAhead = 6;
// 16-dim tiles of O^T per score wave and per load wave (two of each).
constexpr int kScoreDimTiles = 6;
constexpr int kLoadDimTiles = (kVDim / 16 - 2 * kScoreDimTiles) / 2;

struct __align__(16) Lds {
  uint8_t kv[kBuffers][kBufBytes];
  // P^T in PV B-operand order, by block parity: [parity][head tile][lane]
  // 16 bytes: lane (c, g) of tile t holds head 16t + c, k-index j = key
  // 2(j & 3) + 8(g & 1) + (g >> 1) + 16(j >> 2), bf16.
  uint8_t p[2][4][64][16];
  float alpha[2][kHeadsPerGroup];  // per-head rescale factor of the block, by parity
  float row_sum[kHeadsPerGroup];
  int32_t ring[kRing][kBlock];  // block b at slot b % kRing: record row per key, -1 = padding
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

  // Selected id of key `key` of block b (-1 past the selection), its page
  // and its physical record row (-1 for padding, an id outside [0, n_tokens)
  // or a page outside the cache).
  auto id_at = [&](int bl, int key) -> int32_t {
    const int i = bl * kBlock + key;
    return bl < n_blocks && i < topk ? ids[i] : -1;
  };
  auto page_of = [&](int32_t id) -> int32_t {
    if (!kFp8) return 0;
    return id >= 0 && id < n_tokens ? page_table[id / kPageTokens] : -1;
  };
  auto phys_from = [&](int32_t id, int32_t page) -> int32_t {
    if (id < 0 || id >= n_tokens) return -1;
    if (!kFp8) return id;
    return page >= 0 && page < pages ? (int32_t)((int64_t)page * kPageTokens + id % kPageTokens) : -1;
  };

  // Roles: waves 0 and 1 score (32 heads each, all 32 keys of a block, with
  // 32x32x16 MFMAs) and run the softmax; waves 2 and 3 stage the records
  // (HBM -> registers -> bf16 rows in LDS). All four accumulate O^T for their
  // share of the 512 dims over all 64 heads.
  const bool scorer = wave < 2;
  const int sw = wave & 1;           // score wave: heads 32 sw .. + 31
  const int n = lane & 31;           // score lane: head 32 sw + n
  const int h = lane >> 5;           // score lane: row half
  // Staged record bytes of the load waves (fp8: two sets of kLoads at 0 and
  // kLoads, bf16: one set).
  constexpr int kPool = (kFp8 ? 2 : 1) * F::kLoads;
  v4u pool[kPool];
  // Q^T operands of the score waves (k-step ks: dims 16 ks + 8h), 144
  // registers held in AGPRs: loaded straight into them, and read from
  // there as the B operand of the S MFMAs, so that the score waves' VGPRs
  // hold O^T, S, the softmax state and the operand read-ahead without
  // spilling (in VGPRs, about ten of the 36 operands were reloaded from AGPR
  // spill slots every step).
  constexpr int kQOps = kQkDim / 16;
  v4u q_ops[kQOps];
  float m_run = neg_inf;  // score lane: running max of its head (scaled)
  // Row sums of heads 16 wave + c (P^T against ones; every row alike).
  v4f l_acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // Load role: key kk of each block, quarter j of its record.
  const int kk = 16 * (wave & 1) + (lane >> 2);
  const int j = lane & 3;
  const uint32_t ring_base = (uint32_t)(uintptr_t)&lds.ring[0][0];
  const uint32_t kv_base = (uint32_t)(uintptr_t)&lds.kv[0][0];
  const uint32_t p_base = (uint32_t)(uintptr_t)&lds.p[0][0][0][0];
  auto buf_of = [&](int bl) -> uint32_t { return kv_base + (uint32_t)(bl & (kBuffers - 1)) * kBufBytes; };

  // Per-block base addresses are formed once and hidden from the optimizer
  // (an identity DPP move it cannot see through): otherwise it hoists (lane
  // offset + constant) out of the loop and pays an add per LDS access instead
  // of using the instruction's offset field. Unlike an empty asm statement it
  // does not cut the scheduling region.
  auto lane_base = [](uint32_t buf, uint32_t lane_off) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(buf + lane_off), 0xE4, 0xF, 0xF, false);
  };
  auto row_of = [&](int bl) -> int32_t {
    return bl < n_blocks ? lds_load<int32_t>(ring_base + 4 * (uint32_t)((bl % kRing) * kBlock + kk)) : -1;
  };
  // Block b's record bytes of this lane -> registers. Blocks past the end
  // (and invalid ids) read the zero record, so the load count per block is
  // fixed. fp8 latent loads i cover record bytes 64i + 16j (64 contiguous
  // bytes per key and instruction); bf16 loads 2i + u cover 128i + 32j + 16u.
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

  // Prologue: the rows of blocks 0 .. kRingAhead - 1 into the ring; the load
  // waves then keep it kRingAhead blocks ahead (lane: key kk). The id and
  // page loads are branch-free (clamped addresses, out-of-range results
  // replaced).
  for (int t = threadIdx.x; t < kRingAhead * kBlock; t += kThreads) {
    const int32_t id = id_at(t / kBlock, t % kBlock);
    lds.ring[t / kBlock][t % kBlock] = phys_from(id, page_of(id));
  }
  auto id_load = [&](int bl) -> int32_t {
    const int i = bl * kBlock + kk;
    const bool in = bl < n_blocks && i < topk;
    const int32_t id = ids[in ? i : 0];
    return in ? id : -1;
  };
  auto page_load = [&](int32_t id) -> int32_t {
    if (!kFp8) return 0;
    const bool in = id >= 0 && id < n_tokens;
    const int32_t page = page_table[in ? id / kPageTokens : 0];
    return in ? page : -1;
  };
  // Ring state per step parity: the id and page of the block whose row the
  // step stores, and the id loaded for the block two steps after it.
  int32_t ring_id[2] = {-1, -1}, ring_page[2] = {-1, -1}, id_keep[2] = {-1, -1};
  if (!scorer) {
    id_keep[0] = id_load(kRingAhead);
    id_keep[1] = id_load(kRingAhead + 1);
    ring_page[0] = page_load(id_keep[0]);
    ring_page[1] = page_load(id_keep[1]);
    ring_id[0] = id_load(kRingAhead + 2);
    ring_id[1] = id_load(kRingAhead + 3);
    // The records of blocks 0 and 1 from this lane's own id and page loads,
    // without waiting for the ring.
    const int32_t id0 = id_load(0), id1 = id_load(1);
    fetch(Set0{}, phys_from(id0, page_load(id0)));
    if (kFp8) fetch(Set1{}, phys_from(id1, page_load(id1)));
  }
  __syncthreads();  // ring
  // Q^T of the score wave's heads (72 KiB per work-group), loaded only now:
  // issued at the start, the Q loads of all work-groups would queue ahead of
  // the id and page loads that start the pipeline.
  if (scorer) {
    const uint16_t* qrow = q + ((row * heads + head0 + 32 * sw + n) * kQkDim) + 8 * h;
#pragma unroll
    for (int ks = 0; ks < kQOps; ++ks)
      asm volatile("global_load_dwordx4 %0, %1, off" : "=a"(q_ops[ks]) : "v"(qrow + 16 * ks) : "memory");
    // These loads are outside the compiler's load counting: wait here.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  int32_t phys_next = -1;
  if (!scorer) {
    unpack(Set0{}, buf_of(0));
    fetch(Set0{}, row_of(kLookahead - 1));
    phys_next = row_of(kLookahead);
  }
  lds_barrier();

  // Software pipeline, one barrier per step. Step `it`:
  //   score waves: S(it) = K Q^T of block it, the softmax of block it - 1
  //     (its scores kept in registers from the previous step), the PV
  //     product of block it - 2 for their dims;
  //   load waves: rows of block it + 1 into LDS, records of block
  //     it + kLookahead into registers, the PV product of block it - 2.
  // Each wave thus has matrix work (S, PV) and independent VALU / LDS work
  // (softmax, conversion and row stores) in the same step, which the SIMD
  // runs side by side. Buffers: S reads it, PV reads it - 2, the load waves
  // write it + 1 (last read by PV(it - 3), before the previous barrier): four
  // buffers. P and the rescale factors of block b sit at parity b & 1.
  auto step = [&](int it, auto set, auto parity, auto role, auto parts, auto& o, v16f& s_prev)
                  __attribute__((always_inline)) {
    constexpr bool kScore = decltype(role)::value;
    constexpr int kParts = decltype(parts)::value;
    constexpr bool kS = (kParts & 1) != 0;     // score waves: S(it); load waves: rows of it + 1
    constexpr bool kSoft = (kParts & 2) != 0;  // score waves: softmax(it - 1)
    constexpr bool kPV = (kParts & 4) != 0;    // PV(it - 2)
    constexpr int kM = kScore ? kScoreDimTiles : kLoadDimTiles;

    // ---- the step's first LDS reads, before any wait or branch: block
    // it - 2's rescale factors, block it - 1's padding mask, P^T of the four
    // head tiles (and of this wave's tile for its row sums), the first V^T
    // operands (two ds_read_b64_tr_b16 per 16-dim tile, kAheadV tiles ahead)
    // and the first K operands of S(it).
    const uint32_t par_pv = (uint32_t)(it & 1);
    // Load waves read all their V^T operands up front: their row stores
    // later in the step would otherwise sit ahead of V^T reads in the LDS.
    constexpr int kAheadV = kScore ? 3 : kLoadDimTiles;  // score waves: 2 / 3 / 4 measured 160.36 / 160.11 / 160.41 us
    constexpr int kAheadK = 6;
    float al[4];
    int32_t prow = 0;
    v8bf pb[4], p_own;
    v4s vlo[kAheadV], vhi[kAheadV];
    v4u ka[kAheadK];
    uint32_t vbase = 0, kbase = 0;
    if constexpr (kPV) {
#pragma unroll
      for (int t = 0; t < 4; ++t) al[t] = lds.alpha[par_pv][16 * t + c];
    }
    if constexpr (kScore && kSoft)
      prow = lds_load<int32_t>(ring_base + 4 * (uint32_t)(((it - 1) % kRing) * kBlock + n));
    if constexpr (kPV) {
      if constexpr (kScore) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          pb[t] = as_v8bf(lds_load<v4u>(p_base + par_pv * 4096 + (uint32_t)(t * 64 + lane) * 16));
        p_own = as_v8bf(lds_load<v4u>(p_base + par_pv * 4096 + (uint32_t)(wave * 64 + lane) * 16));
      } else {
        // Load waves: P^T straight into AGPRs (read from there as the MFMA
        // B operand), which frees 20 VGPRs of the role that spills (its
        // AGPR reloads per two steps 43 -> 27; layer -0.3 us). The reads go
        // out before the V^T reads, so any wait that covers a V^T operand
        // covers them too; the explicit wait below states it.
        v4u t4[5];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t addr = p_base + par_pv * 4096 + (uint32_t)(t * 64 + lane) * 16;
          asm volatile("ds_read_b128 %0, %1" : "=a"(t4[t]) : "v"(addr) : "memory");
        }
        const uint32_t own = p_base + par_pv * 4096 + (uint32_t)(wave * 64 + lane) * 16;
        asm volatile("ds_read_b128 %0, %1" : "=a"(t4[4]) : "v"(own) : "memory");
#pragma unroll
        for (int t = 0; t < 4; ++t) pb[t] = as_v8bf(t4[t]);
        p_own = as_v8bf(t4[4]);
      }
      vbase = lane_base(buf_of(it - 2), v_lane);
#pragma unroll
      for (int d = 0; d < kAheadV; ++d) {
        vlo[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(vbase + 32 * d));
        vhi[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(vbase + 32 * d + kHalf));
      }
    }
    if constexpr (kScore && kS) {
      kbase = lane_base(buf_of(it), k_lane);
#pragma unroll
      for (int d = 0; d < kAheadK; ++d) ka[d] = lds_load<v4u>(kbase + 32 * d);
    }

    // The step's two data-dependent checks, placed after some independent
    // work so that their LDS reads have landed: rescale O^T (and the row
    // sums) by block it - 2's factors if any head's running max rose, and
    // turn the padding keys of block it - 1 into -inf before its softmax.
    auto checks = [&]() __attribute__((always_inline)) {
      if constexpr (kPV) {
        bool rescale = false;
#pragma unroll
        for (int t = 0; t < 4; ++t) rescale |= al[t] != 1.0f;
        if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int m = 0; m < kM; ++m) o[t][m] *= al[t];
          l_acc *= lds.alpha[par_pv][16 * wave + c];
        }
      }
      if constexpr (kScore && kSoft) {
        const uint32_t vmask = (uint32_t)__builtin_amdgcn_ballot_w64(h == 0 && prow >= 0);
        if (vmask != 0xFFFFFFFFu) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = score_key(8 * (r >> 2) + 4 * h + (r & 3));
            s_prev[r] = (vmask >> key) & 1u ? s_prev[r] : neg_inf;
          }
        }
      }
    };
    // PV MFMA number k of this step (k < 4 kM: dim tile k / 4, head tile
    // k % 4; k = 4 kM: the row sums of this wave's head tile).
    auto pv_mfma = [&](int k) __attribute__((always_inline)) {
      if (k == 4 * kM) {
        const v4u ones = v4u{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
        l_acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(ones), p_own, l_acc, 0, 0, 0);
        return;
      }
      const int m = k >> 2, t = k & 3;
      const v8bf va = __builtin_bit_cast(
          v8bf, __builtin_shufflevector(vlo[m % kAheadV], vhi[m % kAheadV], 0, 1, 2, 3, 4, 5, 6, 7));
      o[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[t], o[t][m], 0, 0, 0);
      if (t == 3 && m + kAheadV < kM) {
        vlo[m % kAheadV] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(vbase + 32 * (m + kAheadV)));
        vhi[m % kAheadV] =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(vbase + 32 * (m + kAheadV) + kHalf));
      }
    };
    constexpr int kPvMfmas = kPV ? 4 * kM + 1 : 0;

    if constexpr (kScore) {
      // ---- S(it) = K Q^T (32 keys x heads 32 sw .. + 31, 36 k-steps of 16
      // dims, back to back), the PV MFMAs and the softmax of block it - 1 in
      // one instruction stream: each k-step issues its MFMA(s), then a slice
      // of the softmax's VALU work, which runs while the MFMAs execute.
      //
      // Softmax of head 32 sw + n: this lane holds keys score_key(8(r / 4) +
      // 4h + r % 4), the other half (lane ^ 32) the rest. Maxima on raw
      // scores (scale_log2 > 0), so that p = exp2(s * scale_log2 - m) is one
      // FMA and one exp2. Row sums come from the PV product (P^T against a
      // row of ones).
      v16f sa = {};
      float mx = neg_inf, alpha = 1.0f, neg_m = 0.0f;
      uint32_t pk[8];
      const uint32_t par_soft = (uint32_t)((it - 1) & 1);
      auto soft_slice = [&](int ks) __attribute__((always_inline)) {
        if (ks < 8) {
          mx = fmaxf(fmaxf(mx, s_prev[2 * ks]), s_prev[2 * ks + 1]);
        } else if (ks == 8) {
          const uint32_t u = __float_as_uint(mx);
          const auto sw32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
          mx = fmaxf(__uint_as_float(sw32[0]), __uint_as_float(sw32[1])) * scale_log2;
          const bool need = mx > m_run + kRescaleThreshold || (m_run == neg_inf && mx != neg_inf);
          const float m_new = need ? fmaxf(m_run, mx) : m_run;
          // exp2(-inf) = 0 covers the first valid block.
          alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
          m_run = m_new;
          // With no valid key so far every score is -inf and p = 0.
          neg_m = m_run == neg_inf ? 0.0f : -m_run;
        } else if (ks < 17) {
          const int r = 2 * (ks - 9);
          pk[ks - 9] = pack_bf16(__builtin_amdgcn_exp2f(__builtin_fmaf(s_prev[r], scale_log2, neg_m)),
                                 __builtin_amdgcn_exp2f(__builtin_fmaf(s_prev[r + 1], scale_log2, neg_m)));
        } else if (ks == 17) {
          // Both row halves hold the same factor; both write it.
          lds.alpha[par_soft][32 * sw + n] = alpha;
          // P^T -> LDS: registers 4a' .. 4a' + 3 are k-indices 4(a' >> 1) ..
          // +3 of operand slot (c = n % 16, g = 2h + (a' & 1)) of head tile
          // 2 sw + n / 16.
          const uint32_t p_tile = p_base + par_soft * 4096 + (uint32_t)((2 * sw + (n >> 4)) * 64 + (n & 15)) * 16;
#pragma unroll
          for (int ap = 0; ap < 4; ++ap) {
            const int gg = 2 * h + (ap & 1);
            lds_store<v2u>(p_tile + (uint32_t)gg * 256 + 8 * (ap >> 1), v2u{pk[2 * ap], pk[2 * ap + 1]});
          }
        }
      };
      // The first kHead k-steps run S alone (the checks' reads land
      // meanwhile); then PV MFMAs and softmax slices join.
      constexpr int kHead = kS ? 3 : 0;
      constexpr int kBody = kPvMfmas > 18 ? kPvMfmas : 18;
      constexpr int kSteps = kS ? kQkDim / 16 : kBody;
      if constexpr (kHead == 0) checks();
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
        if constexpr (kS) {
          const v8bf a = as_v8bf(ka[ks % kAheadK]);
          if (ks + kAheadK < kQkDim / 16) ka[ks % kAheadK] = lds_load<v4u>(kbase + 32 * (ks + kAheadK));
          sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_v8bf(q_ops[ks]), sa, 0, 0, 0);
        }
        if (kHead > 0 && ks == kHead - 1) checks();
        const int kb = ks - kHead;
        if (kb >= 0 && kb < kPvMfmas) pv_mfma(kb);
        if constexpr (kSoft) {
          if (kb >= 0) soft_slice(kb);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int k = kSteps - kHead; k < kPvMfmas; ++k) pv_mfma(k);
      static_assert(!kS || kQkDim / 16 - kHead >= 18, "softmax slices must fit the S k-steps");
      if constexpr (kS) s_prev = sa;
    } else {
      // ---- rows of block it + 1 (its buffer last held block it - 3) in
      // 32 quarters beside the PV MFMAs; the records of block it +
      // kLookahead into the freed registers.
      const uint32_t rec = kS ? lane_base(buf_of(it + 1), (uint32_t)kk * kRowBytes + 32 * j) : 0;
      const v4u* st = pool + decltype(set)::value;
      auto unpack_round = [&](int i) __attribute__((always_inline)) {
        if (kFp8) {
          const float s_i = __builtin_bit_cast(v4f, st[8])[i >> 1];
          const v4u w = st[i];
          const v4u lo{dequant_pair<false>(w.x, s_i), dequant_pair<true>(w.x, s_i),
                       dequant_pair<false>(w.y, s_i), dequant_pair<true>(w.y, s_i)};
          const v4u hi{dequant_pair<false>(w.z, s_i), dequant_pair<true>(w.z, s_i),
                       dequant_pair<false>(w.w, s_i), dequant_pair<true>(w.w, s_i)};
          lds_store<v4u>(rec + 128 * i, lo);
          lds_store<v4u>(rec + 128 * i + 16, hi);
          if (i == 7) {
            lds_store<v4u>(rec + 2 * kVDim, st[9]);
            lds_store<v4u>(rec + 2 * kVDim + 16, st[10]);
          }
        } else {
          lds_store<v4u>(rec + 128 * i, st[2 * i]);
          lds_store<v4u>(rec + 128 * i + 16, st[2 * i + 1]);
          if (i == 7) {
            lds_store<v4u>(rec + 2 * kVDim, st[16]);
            lds_store<v4u>(rec + 2 * kVDim + 16, st[17]);
          }
        }
      };
      // The rounds in quarters (two conversions each; the row's two 16-byte
      // halves stored after quarters 1 and 3), one quarter after each PV
      // MFMA: a 16-cycle MFMA hides about two VALU instructions, so whole
      // rounds (eight conversions) after every sixth MFMA stalled its pipe.
      v4u part_lo = v4u{0u, 0u, 0u, 0u}, part_hi = v4u{0u, 0u, 0u, 0u};
      auto unpack_quarter = [&](int i, int u) __attribute__((always_inline)) {
        if (kFp8) {
          const float s_i = __builtin_bit_cast(v4f, st[8])[i >> 1];
          const v4u w = st[i];
          if (u == 0) {
            part_lo.x = dequant_pair<false>(w.x, s_i);
            part_lo.y = dequant_pair<true>(w.x, s_i);
          } else if (u == 1) {
            part_lo.z = dequant_pair<false>(w.y, s_i);
            part_lo.w = dequant_pair<true>(w.y, s_i);
            lds_store<v4u>(rec + 128 * i, part_lo);
          } else if (u == 2) {
            part_hi.x = dequant_pair<false>(w.z, s_i);
            part_hi.y = dequant_pair<true>(w.z, s_i);
          } else {
            part_hi.z = dequant_pair<false>(w.w, s_i);
            part_hi.w = dequant_pair<true>(w.w, s_i);
            lds_store<v4u>(rec + 128 * i + 16, part_hi);
            if (i == 7) {
              lds_store<v4u>(rec + 2 * kVDim, st[9]);
              lds_store<v4u>(rec + 2 * kVDim + 16, st[10]);
            }
          }
        } else if (u == 3) {
          unpack_round(i);  // bf16 records: stores only
        }
      };
      checks();
      // P^T of the load waves landed: 20 V^T reads follow them.
      if constexpr (kPV) asm volatile("s_waitcnt lgkmcnt(15)" ::: "memory");
      constexpr int kQuarters = kS ? 32 : 0;
      constexpr int kSteps = kPvMfmas > kQuarters ? kPvMfmas : kQuarters;
#pragma unroll
      for (int k = 0; k < kSteps; ++k) {
        if (k < kPvMfmas) pv_mfma(k);
        if (k < kQuarters) unpack_quarter(k / 4, k % 4);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kS) {
        // Ring: row of block it + kRingAhead (its slot held block it - 2)
        // from its id and page, both landed two steps ago; then the page of
        // block it + kRingAhead + 2 from its id (loaded two steps ago, kept
        // for the row two steps from now) and the id of block it +
        // kRingAhead + 4. Each link of the id -> page -> row chain thus has
        // two steps to land (with one step each, the load waves waited
        // ~640 ticks per step here). These loads go out before the record
        // loads, so that waiting for them waits for nothing the step does not
        // wait for anyway. Loaded values live in one register per step parity
        // and are copied only once landed; the four lanes of a key store the
        // same value.
        constexpr int kP = decltype(parity)::value;
        lds.ring[(it + kRingAhead) % kRing][kk] = phys_from(id_keep[kP], ring_page[kP]);
        id_keep[kP] = ring_id[kP];
        ring_page[kP] = page_load(ring_id[kP]);
        ring_id[kP] = id_load(it + kRingAhead + 4);
        fetch(set, phys_next);
        phys_next = row_of(it + kLookahead + 1);
      }
    }
    lds_barrier();
  };
  using Pre0 = std::integral_constant<int, 1>;   // S / rows only
  using Pre1 = std::integral_constant<int, 3>;   // + softmax
  using Full = std::integral_constant<int, 7>;   // + PV
  using Tail0 = std::integral_constant<int, 6>;  // softmax + PV
  using Tail1 = std::integral_constant<int, 4>;  // PV only
  auto run = [&](auto role) __attribute__((always_inline)) {
    constexpr int kM = decltype(role)::value ? kScoreDimTiles : kLoadDimTiles;
    // O^T: head tile t (heads 16t + c), dims dim0 + 16m + 4g + r.
    v4f o[4][kM];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int m = 0; m < kM; ++m) o[t][m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    v16f s_prev = {};
    using Even = std::integral_constant<int, 0>;
    using Odd = std::integral_constant<int, 1>;
    step(0, Set1{}, Even{}, role, Pre0{}, o, s_prev);
    step(1, Set0{}, Odd{}, role, Pre1{}, o, s_prev);
    // Two blocks per trip so that each register set stays a fixed register set.
    for (int it = 2; it < n_blocks; it += 2) {
      step(it, Set1{}, Even{}, role, Full{}, o, s_prev);
      step(it + 1, Set0{}, Odd{}, role, Full{}, o, s_prev);
    }
    step(n_blocks, Set1{}, Even{}, role, Tail0{}, o, s_prev);
    step(n_blocks + 1, Set0{}, Odd{}, role, Tail1{}, o, s_prev);
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
