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
// Mapping (gfx950, wave64, v_mfma_f32_16x16x32_bf16):
// * Work-group = (query row, 64 heads), 4 waves, one per SIMD (each wave has
//   the whole register file: 256 VGPRs plus AGPRs as spill space). Wave w
//   owns heads 16w .. 16w+16 and walks every selected key, keeping its 16
//   heads of Q (72 VGPRs) and O (16 heads x 512 dims, 128 VGPRs) resident.
//   (32 heads per wave would halve LDS bytes per flop but needs ~400 live
//   registers; the online-softmax rescale keeps O out of AGPRs.)
// * Scores are computed transposed, S^T = K Q^T (keys x heads): the C layout
//   of S^T puts head l%16 and keys 4(l/16)+r in lane l, which is the B-operand
//   layout of O^T += V^T P^T when the 32 keys of a block are ordered
//   (l/16, j) -> key 16(j/4) + 4(l/16) + j%4. The probabilities never leave
//   their lane.
// * The records of a block live once in LDS as bf16 rows of 1152 bytes whose
//   16-byte chunks are XOR-swizzled by the row (chunk ^ (row & 15) for the
//   latent, ^ (row & 7) within the RoPE chunks), so the 16 rows read by a
//   16-lane group hit 16 different bank groups. The V^T operand (8 keys of
//   one dim per lane) is read straight from these rows with
//   ds_read_b64_tr_b16: lane 4j+q of a 16-lane group addresses row key_j,
//   dims d0+4q..+3, and lane i receives dim d0+i of key_0..key_3.
// * Gather: the selected records are copied by LDS DMA (global_load_lds,
//   16 bytes per lane, no registers) into a ring of raw stages kRing blocks
//   ahead, with the wait counts managed explicitly, so the random record
//   reads stay in flight while earlier blocks compute. Each iteration then
//   converts one raw stage into the bf16 block (fp8: one
//   v_cvt_scalef32_pk_bf16_fp8 per two values; e4m3 x power-of-two scale is
//   exact in bf16). Physical rows of the whole selection are resolved once
//   into an LDS table.
// * Online softmax in log2 units with lazy rescaling (only when a block
//   raises the running max by more than 8, so p <= 2^8).
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kQkDim = 576;
constexpr int kVDim = 512;
constexpr int kHeadsPerGroup = 64;
constexpr int kBlock = 32;            // keys per block
constexpr int kRowBytes = kQkDim * 2; // bf16 block row (swizzled chunks)
constexpr int kSteps = kQkDim / 32;   // 18 k-steps of 32 dims
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSelected = 4096;    // rows table capacity per query row
constexpr int kPageTokens = 64;
constexpr float kRescaleThreshold = 8.0f;

template <bool kFp8>
struct Geometry {
  static constexpr int kRecordBytes = kFp8 ? 656 : kRowBytes;
  static constexpr int kChunks = kRecordBytes / 16;           // 41 or 72 per record
  static constexpr int kStageChunks = kBlock * kChunks;       // 1312 or 2304
  static constexpr int kLoadsPerWave = (kStageChunks + kThreads - 1) / kThreads;  // 6 or 9
  static constexpr int kStageBytes = kLoadsPerWave * kThreads * 16;
  static constexpr int kRing = kFp8 ? 4 : 2;
};

template <bool kFp8>
struct __align__(16) Lds {
  uint8_t block[kBlock * kRowBytes];                                 // bf16, swizzled
  uint8_t ring[Geometry<kFp8>::kRing][Geometry<kFp8>::kStageBytes];  // raw records
  int32_t rows[kMaxSelected];  // physical record row per selected position, -1 = padding
};

__device__ __forceinline__ v8bf as_v8bf(uint4 v) { return __builtin_bit_cast(v8bf, v); }
__device__ __forceinline__ v8bf as_v8bf(v4u v) { return __builtin_bit_cast(v8bf, v); }

// Two floats -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){lo, hi}, v2bf));
}

// Position of logical 16-byte chunk j (of 72) in block row `row`.
__device__ __forceinline__ int chunk_slot(int j, int row) {
  return j < 64 ? (j ^ (row & 15)) : 64 + ((j - 64) ^ (row & 7));
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

// Issue the DMA of block `blk` into ring slot `slot`. Every wave issues
// exactly kLoadsPerWave loads per stage (padding and invalid rows read the
// first record), which keeps the vmcnt accounting uniform.
template <bool kFp8>
__device__ __forceinline__ void issue_stage(Lds<kFp8>& lds, const uint8_t* __restrict__ kv,
                                            int64_t blk, int64_t iters, int slot) {
  using G = Geometry<kFp8>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < G::kLoadsPerWave; ++k) {
    const int inst = k * kWaves + wave;
    const int chunk = inst * 64 + lane;
    const uint8_t* src = kv;
    if (blk < iters && chunk < G::kStageChunks) {
      const int r = chunk / G::kChunks;
      const int j = chunk - r * G::kChunks;
      const int32_t row = lds.rows[blk * kBlock + r];
      src = kv + (int64_t)(row >= 0 ? row : 0) * G::kRecordBytes + 16 * j;
    }
    const uint32_t base = (uint32_t)(uintptr_t)(&lds.ring[slot][inst * 64 * 16]);
    dma16(src, __builtin_amdgcn_readfirstlane(base));
  }
}

template <bool kHigh>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t word, float scale) {
  v2bf v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, scale, kHigh);
  return __builtin_bit_cast(uint32_t, v);
}

// Raw stage -> swizzled bf16 block. Thread -> (row = t % 32, part = t / 32).
// Padding slots hold a placeholder record in the ring and become zeros here:
// their probability is 0, but 0 x NaN would still poison the PV product.
template <bool kFp8>
__device__ __forceinline__ void convert_stage(Lds<kFp8>& lds, int slot, int64_t blk) {
  using G = Geometry<kFp8>;
  const int r = threadIdx.x & 31;
  const int part = threadIdx.x >> 5;
  const uint8_t* rec = &lds.ring[slot][r * G::kRecordBytes];
  uint8_t* row = &lds.block[r * kRowBytes];
  if (lds.rows[blk * kBlock + r] < 0) {
    const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(row + 16 * (8 * part + i)) = zero;
    *reinterpret_cast<uint4*>(row + 16 * (64 + part)) = zero;
    return;
  }
  if (kFp8) {
    const float scale = *reinterpret_cast<const float*>(rec + kVDim + 4 * (part >> 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * part + i;  // fp8 chunk: values 16j .. 16j+15
      const uint4 w = *reinterpret_cast<const uint4*>(rec + 16 * j);
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
      uint32_t o[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        o[2 * q] = dequant_pair<false>(words[q], scale);
        o[2 * q + 1] = dequant_pair<true>(words[q], scale);
      }
      *reinterpret_cast<uint4*>(row + 16 * chunk_slot(2 * j, r)) = make_uint4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<uint4*>(row + 16 * chunk_slot(2 * j + 1, r)) =
          make_uint4(o[4], o[5], o[6], o[7]);
    }
    const uint4 rope = *reinterpret_cast<const uint4*>(rec + kVDim + 16 + 16 * part);
    *reinterpret_cast<uint4*>(row + 16 * chunk_slot(64 + part, r)) = rope;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * part + i;
      *reinterpret_cast<uint4*>(row + 16 * chunk_slot(j, r)) =
          *reinterpret_cast<const uint4*>(rec + 16 * j);
    }
    *reinterpret_cast<uint4*>(row + 16 * chunk_slot(64 + part, r)) =
        *reinterpret_cast<const uint4*>(rec + 16 * (64 + part));
  }
}

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
  const int64_t head0 = (int64_t)blockIdx.y * kHeadsPerGroup + 16 * wave;
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

  // Q^T operands: head head0 + c, dims 32ks + 8g .. +8.
  v8bf qb[kSteps];
  {
    const uint16_t* qrow = q + ((row * heads + head0 + c) * kQkDim) + 8 * g;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks)
      qb[ks] = as_v8bf(*reinterpret_cast<const uint4*>(qrow + 32 * ks));
  }
  v4f o[kVDim / 16];
#pragma unroll
  for (int m = 0; m < kVDim / 16; ++m) o[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = neg_inf;
  float l_run = 0.0f;

  // All compiler-visible global loads must be complete before the DMA wait
  // accounting starts; the builtin (vmcnt(0), expcnt/lgkmcnt untouched) also
  // tells the compiler so, which keeps it from re-waiting inside the loop.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  lds_barrier();
#pragma unroll
  for (int s = 0; s < G::kRing; ++s) issue_stage<kFp8>(lds, kv, s, iters, s);

  // Operand addresses. S^T rows c and 16 + c share the swizzle (row & 15 ==
  // c); k-step ks reads logical chunk 4 ks + g, whose slot is
  // 16 (ks >> 2) + 4 ((ks & 3) ^ (c >> 2)) + (g ^ (c & 3)): four base
  // addresses plus an immediate offset cover all 18 k-steps (the two RoPE
  // steps use their own pair). V rows vr and 16 + vr (vr = 4g + jj) read
  // logical chunk 2m + (qq >> 1), at slot 16 (m >> 3) + 2 ((m & 7) ^ (vr >> 1))
  // + ((qq >> 1) ^ (vr & 1)): eight bases.
  const int jj = c >> 2;
  const int qq = c & 3;
  const int vr = 4 * g + jj;
  const uint32_t block_base = (uint32_t)(uintptr_t)lds.block;
  uint32_t kbase[4], rbase[2], vbase[8];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    kbase[t] = block_base + c * kRowBytes + 64 * (t ^ (c >> 2)) + 16 * (g ^ (c & 3));
#pragma unroll
  for (int t = 0; t < 2; ++t)
    rbase[t] = block_base + c * kRowBytes + 16 * (64 + ((4 * t + g) ^ (c & 7)));
#pragma unroll
  for (int t = 0; t < 8; ++t)
    vbase[t] = block_base + vr * kRowBytes + 32 * (t ^ (vr >> 1)) + 16 * ((qq >> 1) ^ (vr & 1)) +
               8 * (qq & 1);
  typedef v4s __attribute__((address_space(3))) * lds_v4s;
  typedef v4u __attribute__((address_space(3))) * lds_u4;
  // Row offset of the second 16-key half of the block.
  constexpr uint32_t kHalf = 16 * kRowBytes;
  auto k_addr = [&](int ks) -> uint32_t {
    return ks < 16 ? kbase[ks & 3] + 256 * (ks >> 2) : rbase[ks - 16];
  };
  auto v_addr = [&](int m) -> uint32_t { return vbase[m & 7] + 256 * (m >> 3); };

  for (int64_t it = 0; it < iters; ++it) {
    const int slot = (int)(it % G::kRing);
    wait_dma<G::kLoadsPerWave*(G::kRing - 1)>();  // this wave's loads of block `it`
    lds_barrier();                                 // everyone's loads landed; block free
    convert_stage<kFp8>(lds, slot, it);
    lds_barrier();
    issue_stage<kFp8>(lds, kv, it + G::kRing, iters, slot);

    // ---- S^T = K Q^T for 32 keys x this wave's 16 heads. Operands run two
    // k-steps ahead of the MFMAs; the scheduling barriers keep that order.
    v4f s0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    v4f s1 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    v4u ka[2][2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      ka[d][0] = *(lds_u4)(uintptr_t)k_addr(d);
      ka[d][1] = *(lds_u4)(uintptr_t)(k_addr(d) + kHalf);
    }
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      const v4u a0 = ka[ks & 1][0];
      const v4u a1 = ka[ks & 1][1];
      if (ks + 2 < kSteps) {
        ka[ks & 1][0] = *(lds_u4)(uintptr_t)k_addr(ks + 2);
        ka[ks & 1][1] = *(lds_u4)(uintptr_t)(k_addr(ks + 2) + kHalf);
      }
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a0), qb[ks], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a1), qb[ks], s1, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- online softmax (log2 domain); lane holds head c, keys 16t+4g+r.
    float x[8];
    float mx = neg_inf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = lds.rows[it * kBlock + 16 * t + 4 * g + r] >= 0;
        const float v = valid ? (t ? s1[r] : s0[r]) * scale_log2 : neg_inf;
        x[4 * t + r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const bool need = mx > m_run + kRescaleThreshold || (m_run == neg_inf && mx != neg_inf);
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_run == neg_inf) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int m = 0; m < kVDim / 16; ++m) o[m] *= alpha;
    }
    float p[8];
    const bool live = m_run != neg_inf;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = live ? __builtin_amdgcn_exp2f(x[j] - m_run) : 0.0f;
      l_run += p[j];
    }
    const v8bf pb = as_v8bf(make_uint4(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]),
                                       pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7])));

    // ---- O^T += V^T P^T over 512 dims: dims 16m + 4qq are logical chunk
    // 2m + qq/2 of rows vr and 16 + vr. Transpose loads run kVAhead m-tiles
    // ahead of the MFMAs.
    constexpr int kVAhead = 4;
    v4s vlo[kVAhead], vhi[kVAhead];
#pragma unroll
    for (int d = 0; d < kVAhead; ++d) {
      vlo[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)v_addr(d));
      vhi[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(v_addr(d) + kHalf));
    }
#pragma unroll
    for (int m = 0; m < kVDim / 16; ++m) {
      const v8bf a = __builtin_bit_cast(
          v8bf, __builtin_shufflevector(vlo[m % kVAhead], vhi[m % kVAhead], 0, 1, 2, 3, 4, 5, 6, 7));
      if (m + kVAhead < kVDim / 16) {
        const uint32_t va = v_addr(m + kVAhead);
        vlo[m % kVAhead] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)va);
        vhi[m % kVAhead] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(uintptr_t)(va + kHalf));
      }
      o[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[m], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Drain the DMA issued past the last block (padding loads) before exit.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  const float inv_l = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  // Lane holds head c, dims 16m + 4g + r.
  uint16_t* orow = out + ((row * heads + head0 + c) * kVDim) + 4 * g;
#pragma unroll
  for (int m = 0; m < kVDim / 16; ++m)
    *reinterpret_cast<uint2*>(orow + 16 * m) =
        make_uint2(pack_bf16(o[m][0] * inv_l, o[m][1] * inv_l),
                   pack_bf16(o[m][2] * inv_l, o[m][3] * inv_l));
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
  DSA_CHECK_ARG(pages >= 1 && n_tokens >= 1 && n_tokens <= pages * kPageTokens,
                "page table must cover every token of a nonempty cache");
  DSA_CHECK_ARG(pages * kPageTokens < 0x7FFFFFFF, "cache rows must fit int32");
  DSA_CHECK_ARG(cache && page_table, "null cache or page table");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(cache) % 16 == 0, "cache must be 16-byte aligned");
  return launch<true>(q, rows, heads, cache, page_table, n_tokens, pages, indices, topk, scale,
                      out, stream);
}
