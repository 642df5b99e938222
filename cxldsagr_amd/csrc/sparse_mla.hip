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
// * Work-group = (query row, 64 heads), 8 waves, two per SIMD. Wave w owns
//   heads 16*(w&3) .. +16 of the group and half (w>>2) of the selected keys,
//   so Q=128, H=128 gives 2048 waves, two per SIMD. Each wave keeps its 16
//   heads of Q (72 VGPRs) and its O accumulators (16 heads x 512 dims, 128
//   VGPRs) resident. (32 heads per wave would halve LDS traffic per flop but
//   needs 400 live registers, and the online-softmax rescale of O keeps the
//   accumulators out of AGPRs.)
// * Scores are computed transposed, S^T = K Q^T (keys x heads): the C layout
//   of S^T puts head l%16 and keys 4(l/16)+r in lane l, which is exactly the
//   B-operand layout of O^T += V^T P^T when the 32 keys of a block are
//   ordered (l/16, j) -> key 16(j/4) + 4(l/16) + j%4. The probabilities
//   therefore never leave their lane; V^T is staged in LDS in that key order.
// * Each iteration gathers 64 records (32 per key half) into LDS: K row-major
//   [64][576+8] bf16 (padded stride, conflict-free 16-byte reads) and V^T
//   [2][512][32+8]. fp8 records are dequantised on the way in (e4m3 x
//   power-of-two scale is exact in bf16).
// * Online softmax in log2 units with lazy rescaling: the running max only
//   moves (and O is only rescaled) when a block raises it by more than 8,
//   so p <= 2^8 and the common case skips 256 multiplies per lane.
// * The two key halves are merged with their (max, sum) at the end through
//   LDS, then O / l is rounded to bf16.
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kQkDim = 576;
constexpr int kVDim = 512;
constexpr int kRope = 64;
constexpr int kHeadsPerGroup = 64;
constexpr int kBlock = 32;             // keys per block per key half
constexpr int kKeysPerIter = 2 * kBlock;
constexpr int kKStride = kQkDim + 8;   // bf16 elements per K row in LDS
constexpr int kVtStride = kBlock + 8;  // bf16 elements per V^T row in LDS
constexpr int kSteps = kQkDim / 32;    // 18 k-steps of 32 dims
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kNt = 1;                  // 16-head tiles per wave
constexpr int kRecordFp8 = 656;
constexpr int kPageTokens = 64;
constexpr float kRescaleThreshold = 8.0f;

struct __align__(16) Lds {
  uint16_t k[kKeysPerIter][kKStride];
  uint16_t vt[2][kVDim][kVtStride];
  int32_t valid[kKeysPerIter];
};

// Position of block key k (0..31) in the V^T key order.
__device__ __forceinline__ int vt_slot(int k) {
  const int t = k >> 4, g = (k >> 2) & 3, r = k & 3;
  return 8 * g + 4 * t + r;
}

__device__ __forceinline__ v8bf as_v8bf(uint4 v) { return __builtin_bit_cast(v8bf, v); }

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// Gather the 64 records of this iteration into LDS. Thread -> (key = lane,
// part = wave + 8i), so a wave covers 64 keys at one record offset and the
// transposed V^T stores of a wave are 64 consecutive slots of one row.
template <bool kFp8>
__device__ __forceinline__ void gather_block(Lds& lds, const uint8_t* __restrict__ kv,
                                             const int32_t* __restrict__ page_table,
                                             const int32_t* __restrict__ ids, int64_t n_tokens,
                                             int64_t pages, int64_t topk, int64_t nblk_half,
                                             int64_t it) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int key = lane;
  const int half = key >> 5;
  const int kin = key & 31;
  const int64_t blk = half * nblk_half + it;
  const int64_t pos = blk * kBlock + kin;
  int64_t id = -1;
  if (blk < (half ? 2 * nblk_half : nblk_half) && pos < topk) id = ids[pos];
  bool valid = id >= 0 && id < n_tokens;
  const uint8_t* rec = nullptr;
  if (valid) {
    if (kFp8) {
      // A page number outside the cache is treated like a padding id.
      const int64_t page = page_table[id / kPageTokens];
      valid = page >= 0 && page < pages;
      rec = kv + (page * kPageTokens + id % kPageTokens) * kRecordFp8;
    } else {
      rec = kv + id * (int64_t)(kQkDim * 2);
    }
  }
  if (wave == 0) lds.valid[key] = valid ? 1 : 0;
  const int slot = vt_slot(kin);
  uint16_t* krow = lds.k[key];

  if (kFp8) {
    // 32 latent parts of 16 e4m3 values; tile scale per 8 parts.
#pragma unroll
    for (int i = 0; i < 32 / kWaves; ++i) {
      const int part = wave + kWaves * i;
      uint4 raw = make_uint4(0, 0, 0, 0);
      float scale = 0.0f;
      if (valid) {
        raw = *reinterpret_cast<const uint4*>(rec + part * 16);
        scale = *reinterpret_cast<const float*>(rec + kVDim + 4 * (part >> 3));
      }
      const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t packed[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float v0 = e4m3fn_to_f32(words[w] & 0xFF) * scale;
        float v1 = e4m3fn_to_f32((words[w] >> 8) & 0xFF) * scale;
        float v2 = e4m3fn_to_f32((words[w] >> 16) & 0xFF) * scale;
        float v3 = e4m3fn_to_f32(words[w] >> 24) * scale;
        packed[2 * w] = pack_bf16(v0, v1);
        packed[2 * w + 1] = pack_bf16(v2, v3);
      }
      uint4* dst = reinterpret_cast<uint4*>(krow + part * 16);
      dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        lds.vt[half][part * 16 + e][slot] = (uint16_t)(packed[e >> 1] >> (16 * (e & 1)));
    }
  } else {
#pragma unroll 4
    for (int i = 0; i < 64 / kWaves; ++i) {
      const int part = wave + kWaves * i;
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (valid) raw = *reinterpret_cast<const uint4*>(rec + part * 16);
      *reinterpret_cast<uint4*>(krow + part * 8) = raw;
      const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        lds.vt[half][part * 8 + e][slot] = (uint16_t)(words[e >> 1] >> (16 * (e & 1)));
    }
  }
  // RoPE: 8 parts of 8 bf16.
  const int rope_offset = kFp8 ? kVDim + 16 : kVDim * 2;
#pragma unroll
  for (int i = 0; i < 8 / kWaves; ++i) {
    const int part = wave + kWaves * i;
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (valid) raw = *reinterpret_cast<const uint4*>(rec + rope_offset + part * 16);
    *reinterpret_cast<uint4*>(krow + kVDim + part * 8) = raw;
  }
}

template <bool kFp8>
__global__ __launch_bounds__(kThreads, 1) void sparse_mla_fwd(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kv,
    const int32_t* __restrict__ page_table, int64_t n_tokens, int64_t pages,
    const int32_t* __restrict__ indices, int64_t heads, int64_t topk, float scale_log2,
    uint16_t* __restrict__ out) {
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = wave >> 2;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int64_t row = blockIdx.x;
  const int64_t head0 = (int64_t)blockIdx.y * kHeadsPerGroup + 16 * kNt * (wave & 3);
  const int32_t* ids = indices + row * topk;
  const float neg_inf = -__builtin_inff();

  // Q^T operands: head 16n + c, dims 32ks + 8g .. +8.
  v8bf qb[kNt][kSteps];
#pragma unroll
  for (int n = 0; n < kNt; ++n) {
    const uint16_t* qrow = q + ((row * heads + head0 + 16 * n + c) * kQkDim) + 8 * g;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks)
      qb[n][ks] = as_v8bf(*reinterpret_cast<const uint4*>(qrow + 32 * ks));
  }

  v4f o[kVDim / 16][kNt];
#pragma unroll
  for (int m = 0; m < kVDim / 16; ++m)
#pragma unroll
    for (int n = 0; n < kNt; ++n) o[m][n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[kNt], l_run[kNt];
#pragma unroll
  for (int n = 0; n < kNt; ++n) {
    m_run[n] = neg_inf;
    l_run[n] = 0.0f;
  }

  const int64_t nblk = (topk + kBlock - 1) / kBlock;
  const int64_t nblk_half = (nblk + 1) / 2;
  const int kbase = half * kBlock;

  for (int64_t it = 0; it < nblk_half; ++it) {
    __syncthreads();
    gather_block<kFp8>(lds, kv, page_table, ids, n_tokens, pages, topk, nblk_half, it);
    __syncthreads();

    // ---- S^T = K Q^T for this wave's 32 keys x 32 heads. Operands for the
    // next k-step are loaded while the current one issues; the scheduling
    // barriers stop the compiler from hoisting every LDS load (which would
    // need ~150 extra registers).
    v4f s[2][kNt];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int n = 0; n < kNt; ++n) s[t][n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* krow0 = &lds.k[kbase + c][8 * g];
    const uint16_t* krow1 = &lds.k[kbase + 16 + c][8 * g];
    uint4 a0 = *reinterpret_cast<const uint4*>(krow0);
    uint4 a1 = *reinterpret_cast<const uint4*>(krow1);
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      uint4 n0 = a0, n1 = a1;
      if (ks + 1 < kSteps) {
        n0 = *reinterpret_cast<const uint4*>(krow0 + 32 * (ks + 1));
        n1 = *reinterpret_cast<const uint4*>(krow1 + 32 * (ks + 1));
      }
#pragma unroll
      for (int n = 0; n < kNt; ++n) {
        s[0][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a0), qb[n][ks], s[0][n], 0, 0, 0);
        s[1][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a1), qb[n][ks], s[1][n], 0, 0, 0);
      }
      a0 = n0;
      a1 = n1;
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- online softmax (log2 domain), lane holds head 16n+c, keys 16t+4g+r.
    int valid_bits = 0;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        valid_bits |= lds.valid[kbase + 16 * t + 4 * g + r] << (4 * t + r);

    float x[kNt][8];
    float bmax[kNt];
#pragma unroll
    for (int n = 0; n < kNt; ++n) {
      float mx = neg_inf;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 4 * t + r;
          const float v = ((valid_bits >> j) & 1) ? s[t][n][r] * scale_log2 : neg_inf;
          x[n][j] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      bmax[n] = mx;
    }
    bool need = false;
#pragma unroll
    for (int n = 0; n < kNt; ++n)
      need |= bmax[n] > m_run[n] + kRescaleThreshold || (m_run[n] == neg_inf && bmax[n] != neg_inf);
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
      for (int n = 0; n < kNt; ++n) {
        const float m_new = fmaxf(m_run[n], bmax[n]);
        const float alpha = (m_run[n] == neg_inf) ? 0.0f : exp2f(m_run[n] - m_new);
        m_run[n] = m_new;
        l_run[n] *= alpha;
#pragma unroll
        for (int m = 0; m < kVDim / 16; ++m) o[m][n] *= alpha;
      }
    }
    v8bf pb[kNt];
#pragma unroll
    for (int n = 0; n < kNt; ++n) {
      float p[8];
      const bool live = m_run[n] != neg_inf;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = live ? exp2f(x[n][j] - m_run[n]) : 0.0f;
        l_run[n] += p[j];
      }
      uint4 packed = make_uint4(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]),
                                pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
      pb[n] = as_v8bf(packed);
    }

    // ---- O^T += V^T P^T over 512 dims, one M-tile of 16 dims ahead.
    const uint16_t* vrow = &lds.vt[half][c][8 * g];
    uint4 va = *reinterpret_cast<const uint4*>(vrow);
#pragma unroll
    for (int m = 0; m < kVDim / 16; ++m) {
      uint4 vn = va;
      if (m + 1 < kVDim / 16) vn = *reinterpret_cast<const uint4*>(vrow + 16 * (m + 1) * kVtStride);
#pragma unroll
      for (int n = 0; n < kNt; ++n)
        o[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(va), pb[n], o[m][n], 0, 0, 0);
      va = vn;
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- merge the two key halves: waves 4-7 hand (m, l, O) to waves 0-3.
#pragma unroll
  for (int n = 0; n < kNt; ++n) {
    l_run[n] += __shfl_xor(l_run[n], 16);
    l_run[n] += __shfl_xor(l_run[n], 32);
  }
  constexpr int kStashRegs = kVDim / 16 * kNt * 4 + 2 * kNt;
  static_assert(4 * kStashRegs * 64 * 4 <= (int)sizeof(Lds), "merge stash exceeds LDS");
  __syncthreads();
  float* stash = reinterpret_cast<float*>(&lds) + (wave & 3) * kStashRegs * 64;
  const int mbase = kVDim / 16 * kNt * 4;
  if (half == 1) {
#pragma unroll
    for (int m = 0; m < kVDim / 16; ++m)
#pragma unroll
      for (int n = 0; n < kNt; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) stash[((m * kNt + n) * 4 + r) * 64 + lane] = o[m][n][r];
#pragma unroll
    for (int n = 0; n < kNt; ++n) {
      stash[(mbase + n) * 64 + lane] = m_run[n];
      stash[(mbase + kNt + n) * 64 + lane] = l_run[n];
    }
  }
  __syncthreads();
  if (half == 1) return;
  float a_own[kNt], a_other[kNt], inv_l[kNt];
#pragma unroll
  for (int n = 0; n < kNt; ++n) {
    const float m_other = stash[(mbase + n) * 64 + lane];
    const float l_other = stash[(mbase + kNt + n) * 64 + lane];
    const float m_new = fmaxf(m_run[n], m_other);
    a_own[n] = m_run[n] == neg_inf ? 0.0f : exp2f(m_run[n] - m_new);
    a_other[n] = m_other == neg_inf ? 0.0f : exp2f(m_other - m_new);
    const float l = l_run[n] * a_own[n] + l_other * a_other[n];
    inv_l[n] = l > 0.0f ? 1.0f / l : 0.0f;
  }
  // Lane holds head 16n + c, dims 16m + 4g + r.
#pragma unroll
  for (int n = 0; n < kNt; ++n) {
    uint16_t* orow = out + ((row * heads + head0 + 16 * n + c) * kVDim) + 4 * g;
#pragma unroll
    for (int m = 0; m < kVDim / 16; ++m) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float other = stash[((m * kNt + n) * 4 + r) * 64 + lane];
        v[r] = (o[m][n][r] * a_own[n] + other * a_other[n]) * inv_l[n];
      }
      *reinterpret_cast<uint2*>(orow + 16 * m) =
          make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    }
  }
}

template <bool kFp8>
int launch(const void* q, int64_t rows, int64_t heads, const void* kv, const int32_t* page_table,
           int64_t n_tokens, int64_t pages, const int32_t* indices, int64_t topk, float scale, void* out,
           hipStream_t stream) {
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(sparse_mla_fwd<kFp8>, dim3((unsigned)rows, (unsigned)(heads / kHeadsPerGroup)),
                     dim3(kThreads), 0, stream, static_cast<const uint16_t*>(q),
                     static_cast<const uint8_t*>(kv), page_table, n_tokens, pages, indices, heads, topk,
                     scale_log2, static_cast<uint16_t*>(out));
  DSA_CHECK_LAUNCH("sparse MLA");
  return kOk;
}

int check_common(const void* q, int64_t rows, int64_t heads, const int32_t* indices, int64_t topk,
                 float scale, void* out) {
  DSA_CHECK_ARG(rows >= 0 && topk >= 1, "invalid sparse MLA shape");
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
  DSA_CHECK_ARG(kv_rows >= 0 && kv_rows < 0x7FFFFFFF, "KV row count must fit int32");
  DSA_CHECK_ARG(kv != nullptr || kv_rows == 0, "null kv");
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
  DSA_CHECK_ARG(n_tokens >= 0 && n_tokens <= pages * kPageTokens,
                "page table must cover every token");
  DSA_CHECK_ARG(n_tokens < 0x7FFFFFFF, "token count must fit int32");
  DSA_CHECK_ARG(n_tokens == 0 || (cache && page_table), "null cache or page table");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(cache) % 16 == 0, "cache must be 16-byte aligned");
  return launch<true>(q, rows, heads, cache, page_table, n_tokens, pages, indices, topk, scale,
                      out, stream);
}
