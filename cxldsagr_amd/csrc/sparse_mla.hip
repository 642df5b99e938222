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
// * Scores: wave w computes S^T = K Q^T for key half kh = w / 2 (16 keys)
//   and head half hh = w % 2 (32 heads), keeping Q^T of its 32 heads in
//   AGPRs (144); each K operand read from LDS feeds two MFMAs.
// * Softmax without a max exchange in the common case: each wave computes
//   P against the running max of its heads (known to every wave) and flags
//   the block if any of its maxima rose by more than kRescaleThreshold. If
//   no wave flagged it, P is final. Otherwise (the first block, and rarely
//   later) every wave reads the other key half's block maxima after the
//   barrier, recomputes its P against the new maxima, publishes the rescale
//   factors, and a second barrier precedes the PV product.
// * Values: wave w accumulates O^T for dims 128 w .. 128 w + 127 (one fp8
//   scale tile) and all 64 heads (128 VGPRs). Each V operand feeds four MFMAs.
// * The probabilities, block maxima and flags go through LDS, double
//   buffered by block parity, behind the barrier of the block.
//
// Records travel HBM -> registers -> LDS as bf16 rows. Lane (kk, j) of wave
// w (kk = 8w + lane / 8, j = lane % 8) loads 1/8 of key kk's record of each
// block with 16-byte loads two blocks ahead, and in the iteration before the
// block is scored writes it into one of three row buffers (fp8 records
// converted with their tile scales by v_cvt_scalef32_pk_bf16_fp8; e4m3 x 2^k
// is exact in bf16). Conversion therefore happens once per key, not once
// per wave that reads it, and the score and value phases read plain bf16:
// * K operand: lane (c, g) = (lane % 16, lane / 16) reads 16 bytes of key
//   16 kh + c per k-step.
// * V^T operand: ds_read_b64_tr_b16 - lane 4 jj + qq of a 16-lane row group
//   addresses key 4g + jj at dims d0 + 4qq and receives dim d0 + lane % 16
//   of keys 4g .. 4g + 3 (a second read covers keys 16 + 4g ..).
// A buffer written in iteration b - 1 is read by the scores of block b and,
// after that block's barrier, by its PV product, hence three buffers.
//
// Key order inside a block: MFMA k-index 8g + j of the PV product is key
// 16 (j / 4) + 4g + j % 4, which is where the S^T C layout of the two key
// halves puts them (lane (c, g) holds keys 4g + r of its half, head c).
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
struct Format {
  static constexpr int kRecordBytes = kFp8 ? 656 : kQkDim * 2;
  // 16-byte loads per lane per block: lane (key kk, part j) of the loader
  // fetches 1/8 of its key's record (fp8: 4 latent + scales + RoPE; bf16:
  // 8 latent + RoPE).
  static constexpr int kLoads = kFp8 ? 6 : 9;
};

// bf16 K/V rows of one block in LDS: key r at kRowBytes r, its 576 dims in
// order. The 32-byte pad puts consecutive rows 40 banks apart (mod 64), which
// keeps both the K reads (16 rows x 64 contiguous bytes per half-wave) and
// the V^T transpose reads (8 rows x 32 bytes) free of bank conflicts.
constexpr int kRowBytes = kQkDim * 2 + 32;
constexpr int kBufBytes = kBlock * kRowBytes;
constexpr int kBuffers = 3;  // written in iteration b - 1, read by S in b and by PV after its barrier

struct __align__(16) Lds {
  uint8_t kv[kBuffers][kBufBytes];
  // P^T in PV B-operand order, by block parity: [parity][head tile][lane]
  // 16 bytes, lane (c, g) of tile t holding head 16t + c, keys 4g + r
  // (r = 0..3) then 16 + 4g + r, bf16.
  uint8_t p[2][4][64][16];
  float alpha[2][kHeadsPerGroup];  // per-head rescale factor of the block, by parity
  float part_max[2][2][kHeadsPerGroup];  // [parity][key half] block max of each head
  alignas(16) int32_t raise[2][4];  // [parity][wave]: the block raised a running max
  float row_sum[2][kHeadsPerGroup];  // [key half]
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

// LDS barrier: finish this wave's LDS traffic, then s_barrier. The memory
// clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One block's share of a lane's record bytes, in flight or landed.
template <bool kFp8>
struct Staged {
  v4u r[Format<kFp8>::kLoads];
};

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

  // Physical rows of every selected position.
  for (int i = threadIdx.x; i < n_blocks * kBlock; i += kThreads) {
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

  // Score role: key half kh (keys 16 kh + c), head tiles 2 hh + u (heads
  // 16 (2 hh + u) + c), u = 0, 1.
  const int kh = wave >> 1;
  const int hh = wave & 1;
  // Q^T operands: head 16 (2 hh + u) + c, dims 32 ks + 8g .. +8.
  v8bf qb[2][kSteps];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint16_t* qrow = q + ((row * heads + head0 + 16 * (2 * hh + u) + c) * kQkDim) + 8 * g;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) qb[u][ks] = as_v8bf(*reinterpret_cast<const v4u*>(qrow + 32 * ks));
  }
  // O^T: head tile t (heads 16t + c), dims 128 wave + 16m + 4g + r.
  v4f o[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int m = 0; m < 8; ++m) o[t][m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // Running max of heads 16 (2 hh + u) + c (the same in both key-half
  // waves), and the row sum over this lane's keys.
  float m_run[2] = {neg_inf, neg_inf};
  float l_run[2] = {0.0f, 0.0f};

  // Loader role: key kk of each block, part j of its record.
  const int kk = 8 * wave + (lane >> 3);
  const int j = lane & 7;
  const uint32_t rows_base = (uint32_t)(uintptr_t)&lds.rows[0];
  const uint32_t kv_base = (uint32_t)(uintptr_t)&lds.kv[0][0];
  const uint32_t p_base = (uint32_t)(uintptr_t)&lds.p[0][0][0][0];

  // Block b's record bytes of this lane -> registers. Blocks past the end
  // (and invalid ids) read the zero record, so the load count per block is
  // fixed.
  auto fetch = [&](Staged<kFp8>& st, int b) {
    const int32_t phys = b < n_blocks ? lds_load<int32_t>(rows_base + 4 * (uint32_t)(b * kBlock + kk)) : -1;
    const uint8_t* rec = phys >= 0 ? kv + (int64_t)phys * F::kRecordBytes : zero_record;
    if (kFp8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) st.r[i] = *reinterpret_cast<const v4u*>(rec + 128 * i + 16 * j);
      st.r[4] = *reinterpret_cast<const v4u*>(rec + kVDim);
      st.r[5] = *reinterpret_cast<const v4u*>(rec + kVDim + 16 + 16 * j);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) st.r[i] = *reinterpret_cast<const v4u*>(rec + 128 * i + 16 * j);
      st.r[8] = *reinterpret_cast<const v4u*>(rec + 2 * kVDim + 16 * j);
    }
  };
  // Landed record bytes -> bf16 rows of a block buffer (fp8: e4m3 x tile
  // scale, exact in bf16).
  auto unpack = [&](const Staged<kFp8>& st, uint32_t buf) {
    const uint32_t rec = buf + (uint32_t)kk * kRowBytes;
    if (kFp8) {
      const v4f sc = __builtin_bit_cast(v4f, st.r[4]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4u w = st.r[i];
        const v4u lo{dequant_pair<false>(w.x, sc[i]), dequant_pair<true>(w.x, sc[i]),
                     dequant_pair<false>(w.y, sc[i]), dequant_pair<true>(w.y, sc[i])};
        const v4u hi{dequant_pair<false>(w.z, sc[i]), dequant_pair<true>(w.z, sc[i]),
                     dequant_pair<false>(w.w, sc[i]), dequant_pair<true>(w.w, sc[i])};
        lds_store<v4u>(rec + 256 * i + 32 * j, lo);
        lds_store<v4u>(rec + 256 * i + 32 * j + 16, hi);
      }
      lds_store<v4u>(rec + 2 * kVDim + 16 * j, st.r[5]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) lds_store<v4u>(rec + 128 * i + 16 * j, st.r[i]);
      lds_store<v4u>(rec + 2 * kVDim + 16 * j, st.r[8]);
    }
  };

  // K operand of k-step ks for key 16 kh + c: dims 32 ks + 8g .. +8.
  const uint32_t k_lane = (uint32_t)(16 * kh + c) * kRowBytes + 16 * g;
  // Per-block base addresses are formed once and hidden from the optimizer:
  // otherwise it hoists (lane offset + constant) out of the loop and pays an
  // add per LDS access instead of using the instruction's offset field.
  auto lane_base = [](uint32_t buf, uint32_t lane_off) -> uint32_t {
    uint32_t a = buf + lane_off;
    asm volatile("" : "+v"(a));
    return a;
  };
  // V^T rows (ds_read_b64_tr_b16): lane 4 jj + qq of row group g addresses
  // key vrow = 4g + jj (and 16 + vrow) at dims 128 wave + 16m + 4qq.
  const int jj = c >> 2;
  const int qq = c & 3;
  const int vrow = 4 * g + jj;
  const uint32_t v_lane = (uint32_t)vrow * kRowBytes + 256 * wave + 8 * qq;
  constexpr uint32_t kHalf = 16 * kRowBytes;

  // Prologue: blocks 0 and 1 in flight, block 0 unpacked, block 2 in flight.
  Staged<kFp8> st0, st1;
  __syncthreads();  // rows table
  fetch(st0, 0);
  fetch(st1, 1);
  unpack(st0, kv_base);
  fetch(st0, 2);
  lds_barrier();

  int buf_cur = 0;  // buffer of block it
  // One block: scores, softmax and P of block it; unpack of block it + 1
  // (landed two iterations ago in `st`) and refetch of block it + 3 into it;
  // the barrier; then PV of block it.
  auto step = [&](int it, Staged<kFp8>& st) {
    const uint32_t buf = kv_base + (uint32_t)buf_cur * kBufBytes;
    const uint32_t kbase = lane_base(buf, k_lane);
    const int buf_next_i = buf_cur + 1 == kBuffers ? 0 : buf_cur + 1;
    const uint32_t buf_next = kv_base + (uint32_t)buf_next_i * kBufBytes;
    const uint32_t parity = (uint32_t)(it & 1);

    // ---- block it + 1 -> bf16 rows (first, so that the row writes drain
    // during the score MFMAs); block it + 3 -> the freed registers. The
    // buffer of block it + 1 last held block it - 2, whose readers all passed
    // the previous barrier.
    unpack(st, buf_next);
    fetch(st, it + 3);

    // ---- S^T = K Q^T: keys 16 kh .. +16 x heads of tiles 2 hh, 2 hh + 1;
    // each K operand feeds both head tiles; two accumulators per tile (even /
    // odd k-steps).
    v4f sa[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 2; ++e) sa[u][e] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    {
      constexpr int kAhead = 8;  // K reads in flight (LDS latency under load)
      auto k_addr = [&](int ks) -> uint32_t { return kbase + (uint32_t)(64 * ks); };
      v4u ka[kAhead];
#pragma unroll
      for (int d = 0; d < kAhead; ++d) ka[d] = lds_load<v4u>(k_addr(d));
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
        const v8bf a = as_v8bf(ka[ks % kAhead]);
        if (ks + kAhead < kSteps) ka[ks % kAhead] = lds_load<v4u>(k_addr(ks + kAhead));
        mfma_qb(sa[0][ks & 1], a, qb[0][ks]);
        mfma_qb(sa[1][ks & 1], a, qb[1][ks]);
      }
    }

    // Operands of the softmax, issued before the MFMA results are read.
    const v4i valid = lds_load<v4i>(rows_base + 4 * (uint32_t)(it * kBlock + 16 * kh + 4 * g));
    mfma_drain(sa[0][0], sa[0][1], sa[1][0], sa[1][1]);

    // ---- softmax, speculatively against the running max: lane (c, g) holds
    // keys 16 kh + 4g + r of heads 16 (2 hh + u) + c. If no wave sees a block
    // max above its running max + kRescaleThreshold, the running maxima stand
    // and P is final; otherwise every wave redoes its part after the barrier.
    float x[2][4];
    float mx[2];
    bool raise = false;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const v4f sum = sa[u][0] + sa[u][1];
      mx[u] = neg_inf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[u][r] = valid[r] >= 0 ? sum[r] * scale_log2 : neg_inf;
        mx[u] = fmaxf(mx[u], x[u][r]);
      }
      mx[u] = max_across_rows(mx[u]);
      raise |= mx[u] > m_run[u] + kRescaleThreshold || (m_run[u] == neg_inf && mx[u] != neg_inf);
    }
    const uint32_t p_own = p_base + parity * 4096 + (uint32_t)((2 * hh) * 64 + lane) * 16 + 8 * kh;
    float block_sum[2];
    auto write_p = [&](const float (&mref)[2]) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float pu[4];
        block_sum[u] = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // exp2(-inf) = 0 covers invalid keys; a head with no valid key yet
          // has p = 0.
          pu[r] = mref[u] == neg_inf ? 0.0f : __builtin_amdgcn_exp2f(x[u][r] - mref[u]);
          block_sum[u] += pu[r];
        }
        lds_store<v2u>(p_own + (uint32_t)u * 1024, v2u{pack_bf16(pu[0], pu[1]), pack_bf16(pu[2], pu[3])});
      }
    };
    write_p(m_run);
    if (g == 0) {
      lds.part_max[parity][kh][16 * (2 * hh) + c] = mx[0];
      lds.part_max[parity][kh][16 * (2 * hh + 1) + c] = mx[1];
    }
    if (lane == 0) lds.raise[parity][wave] = __builtin_amdgcn_ballot_w64(raise) != 0;

    lds_barrier();  // P, maxima, flags and block it + 1's rows visible

    // ---- a raised running max: new maxima from both key halves, P again,
    // and the rescale factors of all 64 heads before the PV product.
    const v4i raised = lds_load<v4i>((uint32_t)(uintptr_t)&lds.raise[parity][0]);
    if ((raised.x | raised.y | raised.z | raised.w) != 0) {
      float m_new[2], alpha[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float other = lds.part_max[parity][kh ^ 1][16 * (2 * hh + u) + c];
        m_new[u] = fmaxf(m_run[u], fmaxf(mx[u], other));
        // exp2(-inf) = 0 also covers the first block with a valid key.
        alpha[u] = m_new[u] == neg_inf ? 1.0f : __builtin_amdgcn_exp2f(m_run[u] - m_new[u]);
        m_run[u] = m_new[u];
        l_run[u] *= alpha[u];
      }
      write_p(m_run);
      if (kh == 0 && g == 0) {
        lds.alpha[parity][16 * (2 * hh) + c] = alpha[0];
        lds.alpha[parity][16 * (2 * hh + 1) + c] = alpha[1];
      }
      lds_barrier();
      float al[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) al[t] = lds.alpha[parity][16 * t + c];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int m = 0; m < 8; ++m) o[t][m] *= al[t];
    }
    l_run[0] += block_sum[0];
    l_run[1] += block_sum[1];

    // ---- O^T += V^T P^T for dims 128 wave + (0..127), all 64 heads.
    v8bf pb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      pb[t] = as_v8bf(lds_load<v4u>(p_base + parity * 4096 + (uint32_t)(t * 64 + lane) * 16));
    const uint32_t vbase = lane_base(buf, v_lane);
    auto v_addr = [&](int m) -> uint32_t { return vbase + 32 * m; };
    constexpr int kAhead = 4;
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
    }
    buf_cur = buf_next_i;
  };
  // Two blocks per trip so that each register set stays a fixed register set.
  for (int it = 0; it < n_blocks; it += 2) {
    step(it, st1);
    step(it + 1, st0);
  }
  // The fetches past the last block are never read; let them land before
  // the registers are released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- row sums of all 64 heads (both key halves), then O / l.
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float l = l_run[u];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (g == 0) lds.row_sum[kh][16 * (2 * hh + u) + c] = l;
  }
  __syncthreads();
  uint16_t* obase = out + ((row * heads + head0 + c) * kVDim) + 128 * wave + 4 * g;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float lt = lds.row_sum[0][16 * t + c] + lds.row_sum[1][16 * t + c];
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
