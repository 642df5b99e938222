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
//   streamed from LDS; one instruction is a full 128-deep dot product.
// * C layout: lane l, register r -> head 16t + 4(l/16) + r, key l%16. The
//   head-weighted ReLU sum is 16 in-lane FMAs per key per query; the four
//   lane groups are then combined with a 2-step reduce-scatter so lane l ends
//   with key l of a 64-key stage, giving one coalesced 256-byte row store.
// * Work-group: 8 waves x 2 queries = 16 queries; key range split so the
//   grid is about one work-group per CU. Work-groups that share a key range
//   have block ids 8 apart when the split count is a multiple of 8, so they
//   land on the same XCD and share its L2.
// * K stages of 64 keys x 128 B are double-buffered through LDS with an XOR
//   swizzle of the 16-byte chunks (chunk ^ (key & 7)) against bank conflicts.
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kHeads = 64;
constexpr int kDim = 128;
constexpr int kWaves = 8;
constexpr int kQueriesPerWave = 2;
constexpr int kQueriesPerBlock = kWaves * kQueriesPerWave;
constexpr int kStageKeys = 64;
constexpr int kThreads = kWaves * 64;

__device__ __forceinline__ v8i load_operand(const uint8_t* p) {
  uint4 a = *reinterpret_cast<const uint4*>(p);
  uint4 b = *reinterpret_cast<const uint4*>(p + 16);
  v8i r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  return r;
}

// part[u] holds lane-group partial sums for key (16u + l%16). Returns the
// full sum for key l of the stage.
__device__ __forceinline__ float reduce_scatter4(const float part[4], int group) {
  const bool low = group < 2;
  float send0 = low ? part[2] : part[0];
  float send1 = low ? part[3] : part[1];
  float a0 = (low ? part[0] : part[2]) + __shfl_xor(send0, 32);
  float a1 = (low ? part[1] : part[3]) + __shfl_xor(send1, 32);
  const bool even = (group & 1) == 0;
  float send = even ? a1 : a0;
  return (even ? a0 : a1) + __shfl_xor(send, 16);
}

__global__ __launch_bounds__(kThreads, 1) void logits_fp8_mfma(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ k, const float* __restrict__ w,
    const float* __restrict__ kscale, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ ends, int64_t query_start, int64_t rows, int64_t columns,
    int64_t ldo, int64_t keys_per_split, float* __restrict__ out) {
  __shared__ __align__(16) uint8_t lds_k[2][kStageKeys * kDim];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int group = lane >> 4;
  const int col = lane & 15;
  const int64_t q0 = (int64_t)blockIdx.y * kQueriesPerBlock;
  const int64_t kb = (int64_t)blockIdx.x * keys_per_split;
  const int64_t ke = kb + keys_per_split < ldo ? kb + keys_per_split : ldo;
  const float neg_inf = -__builtin_inff();

  // Largest causal end among this block's queries: keys at or beyond it
  // are -inf for every row and need no MFMA work.
  int64_t max_end = 0;
  for (int i = 0; i < kQueriesPerBlock; ++i) {
    const int64_t qi = q0 + i;
    if (qi < rows) {
      int64_t e = ends ? (int64_t)ends[qi] : query_start + qi + 1;
      max_end = e > max_end ? e : max_end;
    }
  }
  if (max_end > columns) max_end = columns;
  const int64_t kend = ke < max_end ? ke : max_end;
  const int64_t stages = kend > kb ? (kend - kb + kStageKeys - 1) / kStageKeys : 0;

  // Per-wave query operands and weights.
  v8i qa[kQueriesPerWave][4];
  float wt[kQueriesPerWave][16];
  int64_t qrow[kQueriesPerWave];
  int64_t qs[kQueriesPerWave], qe[kQueriesPerWave];
  bool qlive[kQueriesPerWave];
#pragma unroll
  for (int j = 0; j < kQueriesPerWave; ++j) {
    const int64_t qi = q0 + wave * kQueriesPerWave + j;
    qrow[j] = qi;
    qlive[j] = qi < rows;
    const int64_t qc = qlive[j] ? qi : 0;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      qa[j][t] = load_operand(q + ((qc * kHeads + 16 * t + col) * kDim + 32 * group));
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        wt[j][4 * t + r] = qlive[j] ? w[qc * kHeads + 16 * t + 4 * group + r] : 0.0f;
    qs[j] = starts ? (int64_t)starts[qc] : 0;
    qe[j] = ends ? (int64_t)ends[qc] : query_start + qc + 1;
    if (qe[j] > columns) qe[j] = columns;
  }

  // Stage loader: thread -> (key tid/8, 16-byte chunk tid%8).
  const int lkey = tid >> 3;
  const int lchunk = tid & 7;
  const int lds_store_off = lkey * kDim + ((lchunk ^ (lkey & 7)) << 4);
  auto gload = [&](int64_t key0) -> uint4 {
    const int64_t key = key0 + lkey;
    if (key < columns) return *reinterpret_cast<const uint4*>(k + key * kDim + lchunk * 16);
    return make_uint4(0, 0, 0, 0);
  };

  if (stages > 0) {
    uint4 v = gload(kb);
    *reinterpret_cast<uint4*>(&lds_k[0][lds_store_off]) = v;
  }
  __syncthreads();

  for (int64_t s = 0; s < stages; ++s) {
    const int64_t key0 = kb + s * kStageKeys;
    const int buf = (int)(s & 1);
    uint4 next = make_uint4(0, 0, 0, 0);
    if (s + 1 < stages) next = gload(key0 + kStageKeys);

    float part[kQueriesPerWave][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int key = 16 * u + col;
      const uint8_t* base = &lds_k[buf][key * kDim];
      const int c0 = (2 * group) ^ (key & 7);
      const int c1 = (2 * group + 1) ^ (key & 7);
      uint4 lo = *reinterpret_cast<const uint4*>(base + (c0 << 4));
      uint4 hi = *reinterpret_cast<const uint4*>(base + (c1 << 4));
      v8i b;
      b[0] = lo.x; b[1] = lo.y; b[2] = lo.z; b[3] = lo.w;
      b[4] = hi.x; b[5] = hi.y; b[6] = hi.z; b[7] = hi.w;
#pragma unroll
      for (int j = 0; j < kQueriesPerWave; ++j) {
        v4f acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
          acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[j][t], b, zero, 0, 0, 0,
                                                                    0, 0, 0);
        }
        float p = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) p = fmaf(fmaxf(acc[t][r], 0.0f), wt[j][4 * t + r], p);
        part[j][u] = p;
      }
    }

    const int64_t key = key0 + lane;
    const float ks = key < columns ? kscale[key] : 0.0f;
#pragma unroll
    for (int j = 0; j < kQueriesPerWave; ++j) {
      const float total = reduce_scatter4(part[j], group);
      if (qlive[j] && key < ke) {
        const bool visible = key >= qs[j] && key < qe[j];
        out[qrow[j] * ldo + key] = visible ? total * ks : neg_inf;
      }
    }

    if (s + 1 < stages) *reinterpret_cast<uint4*>(&lds_k[buf ^ 1][lds_store_off]) = next;
    __syncthreads();
  }

  // Columns of this split at or beyond every causal end: -inf.
  const int64_t tail = kb + stages * kStageKeys;
  if (tail < ke) {
    for (int i = wave; i < kQueriesPerBlock; i += kWaves) {
      const int64_t qi = q0 + i;
      if (qi >= rows) continue;
      for (int64_t key = tail + lane; key < ke; key += 64) out[qi * ldo + key] = neg_inf;
    }
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_indexer_logits_fp8(const void* q, const void* k, const float* weights,
                                      const float* kscale, const int32_t* starts,
                                      const int32_t* ends, int64_t query_start, int64_t rows,
                                      int64_t columns, int64_t ldo, float* out,
                                      hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(rows >= 0 && columns >= 1, "logits requires nonempty K");
  DSA_CHECK_ARG(ldo >= columns, "output row stride must cover every column");
  DSA_CHECK_ARG(query_start >= 0 && query_start + rows <= columns,
                "query_start must place all query rows inside the visible KV sequence");
  DSA_CHECK_ARG((starts == nullptr) == (ends == nullptr), "starts and ends go together");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(q && k && weights && kscale && out, "null pointer");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(k) % 16 == 0,
                "q and k must be 16-byte aligned");
  const int64_t qgroups = (rows + kQueriesPerBlock - 1) / kQueriesPerBlock;
  const int64_t cus = device_cu_count();
  int64_t splits = (cus + qgroups - 1) / qgroups;
  if (splits < 1) splits = 1;
  int64_t per = (ldo + splits - 1) / splits;
  per = (per + kStageKeys - 1) / kStageKeys * kStageKeys;
  splits = (ldo + per - 1) / per;
  DSA_CHECK_ARG(qgroups < 65536, "too many query rows for one launch");
  hipLaunchKernelGGL(logits_fp8_mfma, dim3((unsigned)splits, (unsigned)qgroups), dim3(kThreads),
                     0, stream, static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k),
                     weights, kscale, starts, ends, query_start, rows, columns, ldo, per, out);
  DSA_CHECK_LAUNCH("indexer logits");
  return kOk;
}
