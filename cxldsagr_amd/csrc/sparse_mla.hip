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
// Mapping (gfx950, wave64, v_mfma_f32_16x16x32_bf16). A work-group owns one
// query row and 64 heads and walks the selection in blocks of 32 keys; its 4
// waves (one per SIMD) split each block twice:
// * Scores: wave w computes S^T = K Q^T for all 32 keys (two 16-key tiles)
//   and its 16 heads 16 w .. 16 w + 15, keeping Q^T of those heads in AGPRs
//   (72). The block max of a head is then a reduction inside the wave, and
//   the wave owns the running max, rescale factor and row sum of its heads.
// * Values: wave w accumulates O^T for dims 128 w .. 128 w + 127 (one fp8
//   scale tile) and all 64 heads (128 VGPRs). Each V operand feeds four MFMAs.
// * The probabilities and per-head rescale factors go through LDS, double
//   buffered by block parity, behind the one barrier of the block. That
//   barrier also publishes the next block's records and frees the ring slot
//   of the previous block.
// Records reach LDS by LDS DMA (global_load_lds_dwordx4: 16 bytes per lane,
// no registers) into a ring of raw stages kRing - 1 blocks ahead, with the
// wait counts managed explicitly. A block's loads are issued in three parts
// spread over the PV product (a full memory queue stalls the issuing wave),
// and the first score operands of block it + 1 are read right after the
// barrier. fp8 records are consumed raw:
// * K operand: lane (c, g) = (lane % 16, lane / 16) reads 8 e4m3 of key c and
//   converts them with the key's tile scale (v_cvt_scalef32_pk_bf16_fp8;
//   e4m3 x 2^k is exact in bf16).
// * V^T operand: ds_read_b64_tr_b8 - within a 16-lane group, lane 8q + b
//   receives byte b of the 8-byte segments addressed by lanes 2j + q,
//   j = 0..7. Lanes 2j + q address key j at dims d0 + 8q, so lane i gets dim
//   d0 + i of 8 keys: the A operand of O^T += V^T P^T after an unscaled
//   conversion. The per-key scale of the wave's tile is folded into P
//   (P x 2^k is exact in bf16), so the score waves write one P copy per dim
//   tile.
// bf16 records are DMA'd straight into rows whose 16-byte chunks are
// XOR-swizzled by the key (chunk ^ (key & 15) for the latent, ^ (key & 7)
// within the RoPE chunks); V^T then comes from ds_read_b64_tr_b16.
//
// Key order inside a block: MFMA k-index 8g + j of the PV product is key
// 16 (j / 4) + 4g + j % 4, which is where the S^T C layout of the two key
// tiles puts them (lane (c, g) holds keys 4g + r of each tile, head c).
//
// Online softmax in log2 units with lazy rescaling (only when a block raises
// the running max by more than 8, so p <= 2^8).
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
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));

constexpr int kQkDim = 576;
constexpr int kVDim = 512;
constexpr int kHeadsPerGroup = 64;
constexpr int kBlock = 32;            // keys per block
constexpr int kSteps = kQkDim / 32;   // 18 k-steps of 32 dims
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSelected = 4096;    // rows table capacity per query row
constexpr int kPageTokens = 64;
constexpr float kRescaleThreshold = 8.0f;

template <bool kFp8>
struct Geometry {
  static constexpr int kRecordBytes = kFp8 ? 656 : kQkDim * 2;
  static constexpr int kChunks = kRecordBytes / 16;  // 41 or 72 per record
  // fp8: record r at chunk 41 r, plus 8 chunks (128 bytes) for the second
  // key half. 8-byte LDS reads are served 32 lanes at a time from 64 4-byte
  // banks; with the 656-byte stride alone, keys r and r + 16 share banks, and
  // the V^T reads of one cycle (keys 0-7 and 16-23, or 8-15 and 24-31) would
  // conflict. The shift moves the second half onto the complementary banks.
  // bf16: record r at chunk 72 r.
  static constexpr int kHalfPad = kFp8 ? 8 : 0;
  static constexpr int kStageChunks = kBlock * kChunks + kHalfPad;
  static constexpr int kLoadsPerWave = (kStageChunks + kThreads - 1) / kThreads;  // 6 or 9
  static constexpr int kStageBytes = kLoadsPerWave * kThreads * 16;
  static constexpr int kRing = kFp8 ? 4 : 3;
  static constexpr int kPVersions = kFp8 ? 4 : 1;  // P copies (one per V scale tile)
  __device__ static constexpr uint32_t record_offset(int r) {
    return 16u * (uint32_t)(kChunks * r + (r >= 16 ? kHalfPad : 0));
  }
};

template <bool kFp8>
struct __align__(16) Lds {
  uint8_t ring[Geometry<kFp8>::kRing][Geometry<kFp8>::kStageBytes];  // raw records
  // P^T in PV B-operand order, by block parity: [parity][version][head tile]
  // [lane] 16 bytes, lane (c, g) of tile t holding head 16t + c, keys 4g + r
  // (r = 0..3) then 16 + 4g + r, bf16.
  uint8_t p[2][Geometry<kFp8>::kPVersions][4][64][16];
  float alpha[2][kHeadsPerGroup];  // per-head rescale factor of the block, by parity
  float row_sum[kHeadsPerGroup];
  int32_t rows[kMaxSelected];  // physical record row per selected position, -1 = padding
};

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

// acc += a b for the score MFMAs, with b (Q^T) pinned to AGPRs: Q^T of 32
// heads (144 registers) and the O accumulators (128) do not both fit the 256
// VGPRs, and as a compiler-chosen spill Q^T is copied back into an aligned
// tuple before every use. As inline assembly the MFMA is invisible to the
// hazard recognizer, so it covers its own wait states: the leading s_nop 1
// gives the 2 required after a VALU write of `a` or `acc`; the reader of the
// final accumulators waits with mfma_drain().
__device__ __forceinline__ void mfma_qb(v4f& acc, v8bf a, v8bf b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "a"(b));
}

// Max over the four 16-lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48) with the
// gfx950 row-swap permutes instead of LDS-routed shuffles.
__device__ __forceinline__ float max_across_rows(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(m);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Wait states between the last inline-assembly MFMAs and any read of their
// results (more than the 11 an 8-pass XDL op needs). The accumulators are
// operands, so no read of them can be scheduled above the wait.
__device__ __forceinline__ void mfma_drain(v4f& a, v4f& b, v4f& c, v4f& d) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

// 8 e4m3 (two dwords) x scale -> 8 bf16.
__device__ __forceinline__ v8bf dequant8(v2u w, float scale) {
  return as_v8bf(v4u{dequant_pair<false>(w.x, scale), dequant_pair<true>(w.x, scale),
                     dequant_pair<false>(w.y, scale), dequant_pair<true>(w.y, scale)});
}

// Position of logical 16-byte chunk j (of 72) in bf16 record `key`.
__device__ __forceinline__ int chunk_slot(int j, int key) {
  return j < 64 ? (j ^ (key & 15)) : 64 + ((j - 64) ^ (key & 7));
}

typedef v2i __attribute__((address_space(3))) * lds_v2i;
typedef v4s __attribute__((address_space(3))) * lds_v4s;

template <typename T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
  return *(T __attribute__((address_space(3)))*)(uintptr_t)addr;
}
template <typename T>
__device__ __forceinline__ void lds_store(uint32_t addr, T v) {
  *(T __attribute__((address_space(3)))*)(uintptr_t)addr = v;
}

// LDS barrier that does not wait for the in-flight DMA stages: finish this
// wave's LDS traffic, then s_barrier. The memory clobber keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int kOutstanding>
__device__ __forceinline__ void wait_dma() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kOutstanding) : "memory");
}

// One wave's LDS DMA for 64 consecutive 16-byte chunks of a raw stage: lane l
// copies its chunk to lds_base + 16 l.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               ::"s"(lds_base), "v"(src) : "memory", "m0");
}

// Stage chunk -> (record slot r, logical chunk j) of the DMA source, or r = -1
// for padding.
template <bool kFp8>
__device__ __forceinline__ void stage_chunk(int sc, int& r, int& j) {
  using G = Geometry<kFp8>;
  if (kFp8) {
    constexpr int kHalf = 16 * G::kChunks;
    int base = sc;
    int r0 = 0;
    if (sc >= kHalf) {
      base = sc - kHalf - G::kHalfPad;
      r0 = 16;
    }
    if (base < 0 || base >= kHalf) {
      r = -1;
      j = 0;
      return;
    }
    const int rr = base / G::kChunks;
    r = r0 + rr;
    j = base - rr * G::kChunks;
  } else {
    if (sc >= G::kStageChunks) {
      r = -1;
      j = 0;
      return;
    }
    r = sc / G::kChunks;
    const int p = sc - r * G::kChunks;  // physical slot; the swizzle is an involution
    j = chunk_slot(p, r);
  }
}

// DMA plan of one lane: for each of its kLoadsPerWave loads per stage, the
// record slot r (0xFFFF for padding) and the chunk's byte offset 16 j.
template <bool kFp8>
struct DmaPlan {
  uint32_t rj[Geometry<kFp8>::kLoadsPerWave];  // (r << 16) | 16 j
  int32_t row[Geometry<kFp8>::kLoadsPerWave];  // physical rows of the next block to issue

  __device__ __forceinline__ void init() {
    using G = Geometry<kFp8>;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < G::kLoadsPerWave; ++k) {
      int r, j;
      stage_chunk<kFp8>((k * kWaves + wave) * 64 + lane, r, j);
      rj[k] = r < 0 ? 0xFFFF0000u : ((uint32_t)r << 16) | (uint32_t)(16 * j);
    }
  }
  // Reads the physical rows of block `blk` (-1 where nothing is fetched).
  __device__ __forceinline__ void load_rows(const int32_t* rows, int blk, int n_blocks) {
    using G = Geometry<kFp8>;
#pragma unroll
    for (int k = 0; k < G::kLoadsPerWave; ++k) {
      const uint32_t r = rj[k] >> 16;
      const bool use = blk < n_blocks && r != 0xFFFF;
      const int32_t v = rows[use ? blk * kBlock + (int)r : 0];
      row[k] = use ? v : -1;
    }
  }
  // Issues loads [k0, k1) of the block whose rows were loaded, into the stage
  // at slot_base. Loads without a record read the zero record.
  template <int k0, int k1>
  __device__ __forceinline__ void issue(const uint8_t* __restrict__ kv, const uint8_t* zero,
                                        uint32_t slot_base) const {
    using G = Geometry<kFp8>;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = k0; k < k1; ++k) {
      const bool use = row[k] >= 0;
      const uint8_t* src = (use ? kv : zero) +
                           (use ? (int64_t)row[k] * G::kRecordBytes + (rj[k] & 0xFFFF) : 0);
      dma16(src, __builtin_amdgcn_readfirstlane(slot_base + (k * kWaves + wave) * 64 * 16));
    }
  }
};

template <bool kFp8>
__global__ __launch_bounds__(kThreads, 1) void sparse_mla_fwd(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv,
    const int32_t* __restrict__ page_table, int64_t n_tokens, int64_t pages,
    const int32_t* __restrict__ indices, int64_t heads, int64_t topk, float scale_log2,
    uint16_t* __restrict__ out) {
  using G = Geometry<kFp8>;
  __shared__ Lds<kFp8> lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int64_t row = blockIdx.x;
  const int64_t head0 = (int64_t)blockIdx.y * kHeadsPerGroup;
  const int32_t* ids = indices + row * topk;
  const float neg_inf = -__builtin_inff();
  const int64_t iters = (topk + kBlock - 1) / kBlock;

  // Physical rows of every selected position.
  for (int64_t i = threadIdx.x; i < iters * kBlock; i += kThreads) {
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
    lds.rows[i] = phys;
  }

  // Q^T operands of the score phase: head 16 wave + c, dims 32ks + 8g .. +8.
  v8bf qb[kSteps];
  {
    const uint16_t* qrow = q + ((row * heads + head0 + 16 * wave + c) * kQkDim) + 8 * g;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) qb[ks] = as_v8bf(*reinterpret_cast<const v4u*>(qrow + 32 * ks));
  }
  // O^T: head tile t (heads 16t + c), dims 128 wave + 16m + 4g + r.
  v4f o[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int m = 0; m < 8; ++m) o[t][m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = neg_inf;  // running max of head 16 wave + c
  float l_run = 0.0f;     // its row sum over this lane's keys

  // All compiler-visible global loads must be complete before the DMA wait
  // accounting starts; the builtin (vmcnt(0), expcnt/lgkmcnt untouched) also
  // tells the compiler so, which keeps it from re-waiting inside the loop.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  lds_barrier();
  const uint8_t* zero = zero_record;
  const uint32_t ring_base = (uint32_t)(uintptr_t)&lds.ring[0][0];
  const int n_blocks = (int)iters;
  constexpr int kL = G::kLoadsPerWave;
  DmaPlan<kFp8> dma;
  dma.init();
#pragma unroll
  for (int s = 0; s < G::kRing - 1; ++s) {
    dma.load_rows(lds.rows, s, n_blocks);
    dma.template issue<0, kL>(kv, zero, ring_base + s * G::kStageBytes);
  }
  dma.load_rows(lds.rows, G::kRing - 1, n_blocks);

  const uint32_t p_base = (uint32_t)(uintptr_t)&lds.p[0][0][0][0][0];
  const uint32_t rows_base = (uint32_t)(uintptr_t)&lds.rows[0];
  constexpr uint32_t kPParity = G::kPVersions * 4 * 64 * 16;
  // V^T (tr8) rows: lane 2j + q of each 16-lane group reads key
  // 16 (j / 4) + 4g + j % 4 at dims +8q.
  const int vj = c >> 1;
  const int vq = c & 1;
  const int vkey = 16 * (vj >> 2) + 4 * g + (vj & 3);

  // bf16 K operand of k-step ks: logical chunk 4 ks + g of key 16t + c sits
  // at slot 16 (ks >> 2) + 4 ((ks & 3) ^ (c >> 2)) + (g ^ (c & 3)).
  auto k_addr_bf16 = [&](uint32_t srec, int ks) -> uint32_t {
    return ks < 16 ? srec + 256 * (ks >> 2) + 64 * ((ks & 3) ^ (c >> 2)) + 16 * (g ^ (c & 3))
                   : srec + 16 * (64 + ((4 * (ks - 16) + g) ^ (c & 7)));
  };
  // Score operands of key tiles t = 0, 1 (keys 16t + c), loaded ahead (fp8:
  // the key's tile scales and the first raw K chunks; bf16: the first chunks).
  constexpr int kKAhead = kFp8 ? 4 : 2;
  v4f ksc[2];
  v2u raw[2][kKAhead];
  v4u ka[2][kKAhead];
  auto s_rec = [&](uint32_t stage_k, int t) -> uint32_t {
    return stage_k + G::record_offset(16 * t + c) + (kFp8 ? 8 * g : 0);
  };
  auto prefetch_k = [&](uint32_t stage_k) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t srec = s_rec(stage_k, t);
      if (kFp8) {
        ksc[t] = lds_load<v4f>(srec - 8 * g + kVDim);
#pragma unroll
        for (int d = 0; d < kKAhead; ++d) raw[t][d] = lds_load<v2u>(srec + 32 * d);
      } else {
#pragma unroll
        for (int d = 0; d < kKAhead; ++d) ka[t][d] = lds_load<v4u>(k_addr_bf16(srec, d));
      }
    }
  };
  wait_dma<kL * (G::kRing - 2)>();  // this wave's loads of block 0
  lds_barrier();
  prefetch_k(ring_base);

  int slot = 0;                  // ring slot of block it
  int free_slot = G::kRing - 1;  // slot of block it - 1, refilled with block it + kRing - 1
  for (int it = 0; it < n_blocks; ++it) {
    const uint32_t stage = ring_base + (uint32_t)slot * G::kStageBytes;
    const uint32_t parity = (uint32_t)(it & 1);

    // ---- S^T = K Q^T: keys 0..31 (two 16-key tiles) x heads 16 wave + c;
    // two accumulators per tile (even / odd k-steps).
    v4f sa[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) sa[t][u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (kFp8) {
      v4u rope[2][2];
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t srec = s_rec(stage, t);
          v8bf a;
          if (ks < 16) {
            a = dequant8(raw[t][ks % kKAhead], ksc[t][ks >> 2]);
            if (ks + kKAhead < 16) {
              raw[t][ks % kKAhead] = lds_load<v2u>(srec + 32 * (ks + kKAhead));
            } else if (ks + kKAhead < 18) {
              rope[t][ks + kKAhead - 16] = lds_load<v4u>(srec + 8 * g + kVDim + 16 + 64 * (ks + kKAhead - 16));
            }
          } else {
            a = as_v8bf(rope[t][ks - 16]);
          }
          mfma_qb(sa[t][ks & 1], a, qb[ks]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v8bf a = as_v8bf(ka[t][ks % kKAhead]);
          if (ks + kKAhead < kSteps) ka[t][ks % kKAhead] = lds_load<v4u>(k_addr_bf16(s_rec(stage, t), ks + kKAhead));
          mfma_qb(sa[t][ks & 1], a, qb[ks]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // Operands of the softmax, issued before the MFMA results are read.
    v4i valid[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
      valid[t] = lds_load<v4i>(rows_base + 4 * (uint32_t)(it * kBlock + 16 * t + 4 * g));
    v4f vsc[2][4];  // fp8: tile scales of keys 16t + 4g + r
    if (kFp8) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) vsc[t][r] = lds_load<v4f>(stage + G::record_offset(16 * t + 4 * g + r) + kVDim);
    }
    mfma_drain(sa[0][0], sa[0][1], sa[1][0], sa[1][1]);

    // ---- online softmax of head 16 wave + c over the whole block (lane
    // (c, g) holds keys 16t + 4g + r; the max over g uses the row-swap permutes).
    float x[2][4];
    float mx = neg_inf;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const v4f sum = sa[t][0] + sa[t][1];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[t][r] = valid[t][r] >= 0 ? sum[r] * scale_log2 : neg_inf;
        mx = fmaxf(mx, x[t][r]);
      }
    }
    mx = max_across_rows(mx);
    const bool need = mx > m_run + kRescaleThreshold || (m_run == neg_inf && mx != neg_inf);
    const float m_new = need ? fmaxf(m_run, mx) : m_run;
    // exp2(-inf) = 0 covers the first valid block.
    const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    m_run = m_new;
    l_run *= alpha;
    float p[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[t][r] = m_run == neg_inf ? 0.0f : __builtin_amdgcn_exp2f(x[t][r] - m_run);
        l_run += p[t][r];
      }
    if (g == 0) lds.alpha[parity][16 * wave + c] = alpha;
    // P^T -> LDS, one copy per V scale tile for fp8 (scaled by each key's
    // scale of that tile; P x 2^k is exact in bf16).
    const uint32_t p_own = p_base + parity * kPParity + (uint32_t)(wave * 64 + lane) * 16;
    if (kFp8) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const v4u pk{pack_bf16(p[0][0] * vsc[0][0][v], p[0][1] * vsc[0][1][v]),
                     pack_bf16(p[0][2] * vsc[0][2][v], p[0][3] * vsc[0][3][v]),
                     pack_bf16(p[1][0] * vsc[1][0][v], p[1][1] * vsc[1][1][v]),
                     pack_bf16(p[1][2] * vsc[1][2][v], p[1][3] * vsc[1][3][v])};
        lds_store<v4u>(p_own + (uint32_t)v * 4096, pk);
      }
    } else {
      const v4u pk{pack_bf16(p[0][0], p[0][1]), pack_bf16(p[0][2], p[0][3]),
                   pack_bf16(p[1][0], p[1][1]), pack_bf16(p[1][2], p[1][3])};
      lds_store<v4u>(p_own, pk);
    }

    // Block it + 1's records: this wave's loads first, then the barrier
    // makes everyone's visible, publishes P and alpha, and (every wave having
    // finished PV of block it - 1) frees the slot of block it - 1.
    wait_dma<kL * (G::kRing - 3)>();
    lds_barrier();
    const uint32_t fill = ring_base + (uint32_t)free_slot * G::kStageBytes;
    dma.template issue<0, kL / 3>(kv, zero, fill);
    slot = slot + 1 == G::kRing ? 0 : slot + 1;
    free_slot = free_slot + 1 == G::kRing ? 0 : free_slot + 1;
    if (it + 1 < n_blocks) prefetch_k(ring_base + (uint32_t)slot * G::kStageBytes);

    // ---- O^T += V^T P^T for dims 128 wave + (0..127), all 64 heads.
    float al[4];
    bool rescale = false;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      al[t] = lds.alpha[parity][16 * t + c];
      rescale |= al[t] != 1.0f;
    }
    if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int m = 0; m < 8; ++m) o[t][m] *= al[t];
    }
    v8bf pb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      pb[t] = as_v8bf(lds_load<v4u>(p_base + parity * kPParity +
                                    (uint32_t)(((kFp8 ? wave : 0) * 4 + t) * 64 + lane) * 16));
    if (kFp8) {
      const uint32_t vaddr = stage + G::record_offset(vkey) + 128 * wave + 8 * vq;
      constexpr int kAhead = 3;
      v2u vr[kAhead];
#pragma unroll
      for (int d = 0; d < kAhead; ++d)
        vr[d] = __builtin_bit_cast(v2u, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i)(uintptr_t)(vaddr + 16 * d)));
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const v8bf a = dequant8(vr[m % kAhead], 1.0f);
        if (m + kAhead < 8)
          vr[m % kAhead] = __builtin_bit_cast(
              v2u, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i)(uintptr_t)(vaddr + 16 * (m + kAhead))));
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[t], o[t][m], 0, 0, 0);
        if (m == 2) dma.template issue<kL / 3, 2 * kL / 3>(kv, zero, fill);
        if (m == 5) dma.template issue<2 * kL / 3, kL>(kv, zero, fill);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // Dims 16 mg + 4 qq of rows vrow and 16 + vrow (vrow = 4g + jj): logical
      // chunk 2 mg + (qq >> 1), slot 16 (mg >> 3) + 2 ((mg & 7) ^ (vrow >> 1)) +
      // ((qq >> 1) ^ (vrow & 1)), with mg = 8 wave + m.
      const int jj = c >> 2;
      const int qq = c & 3;
      const int vrow = 4 * g + jj;
      const uint32_t vbase = stage + G::record_offset(vrow) + 256 * wave +
                             16 * ((qq >> 1) ^ (vrow & 1)) + 8 * (qq & 1);
      constexpr uint32_t kHalf = 16 * G::kRecordBytes;
      auto v_addr = [&](int m) -> uint32_t { return vbase + 32 * (m ^ (vrow >> 1)); };
      constexpr int kAhead = 3;
      v4s vlo[kAhead], vhi[kAhead];
#pragma unroll
      for (int d = 0; d < kAhead; ++d) {
        vlo[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)v_addr(d));
        vhi[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(v_addr(d) + kHalf));
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const v8bf a = __builtin_bit_cast(
            v8bf, __builtin_shufflevector(vlo[m % kAhead], vhi[m % kAhead], 0, 1, 2, 3, 4, 5, 6, 7));
        if (m + kAhead < 8) {
          vlo[m % kAhead] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)v_addr(m + kAhead));
          vhi[m % kAhead] =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(v_addr(m + kAhead) + kHalf));
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[t], o[t][m], 0, 0, 0);
        if (m == 2) dma.template issue<kL / 3, 2 * kL / 3>(kv, zero, fill);
        if (m == 5) dma.template issue<2 * kL / 3, kL>(kv, zero, fill);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    dma.load_rows(lds.rows, it + G::kRing, n_blocks);  // rows of the next refill
  }
  // Drain the DMA issued past the last block (padding loads) before exit.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- row sums of all 64 heads, then O / l.
  float l = l_run;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (g == 0) lds.row_sum[16 * wave + c] = l;
  __syncthreads();
  uint16_t* obase = out + ((row * heads + head0 + c) * kVDim) + 128 * wave + 4 * g;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float lt = lds.row_sum[16 * t + c];
    const float inv_l = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t* orow = obase + (int64_t)16 * t * kVDim;
#pragma unroll
    for (int m = 0; m < 8; ++m)
      *reinterpret_cast<uint2*>(orow + 16 * m) =
          make_uint2(pack_bf16(o[t][m][0] * inv_l, o[t][m][1] * inv_l),
                     pack_bf16(o[t][m][2] * inv_l, o[t][m][3] * inv_l));
  }
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
