// A6: exact top-k (k <= 2048) per row with SMALL tie order.
//
// Semantics: operators/deepseek_v32/indexer/selection.py:62-113 - values in
// descending radix order of their fp32 bits (so -0.0 ranks below +0.0), ties
// resolved to the smaller column, values copied bit-exactly, index -1 where
// the value is inf or NaN (selection.py:43-51).
//
// Every element gets a unique 64-bit composite key
//     K = (radix(v) << 32) | ~column
// whose descending order is exactly the required output order (the same key
// the reference spells out in indexer/csrc/q1_topk_sort.cu:24-42). Selecting
// the top `count` composite keys therefore needs no tie handling at all:
//
// 1. histogram of the top 11 bits over the row (global memory, 1 pass);
// 2. second pass: keys above the threshold bucket go straight to the
//    selected set in LDS, keys in the bucket go to an LDS refine buffer;
// 3. the remaining digits (11/10/11/11/10 bits) are resolved on the LDS
//    buffer; a bucket too large for LDS (huge ties, e.g. masked rows) falls
//    back to further histogram passes over the row;
// 4. bitonic sort of the <= 2048 selected keys in LDS, then values and
//    indices are decoded from the keys.
//
// One 1024-thread work-group per row; the row is read twice from HBM/L2 in
// the common case.
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

constexpr int kThreads = 1024;
constexpr int kBins = 2048;
constexpr int kMaxK = 2048;
constexpr int kRefineCap = 6144;
constexpr int kLevels = 6;
__constant__ int kShift[kLevels] = {53, 42, 32, 21, 10, 0};
__constant__ int kWidth[kLevels] = {11, 11, 10, 11, 11, 10};

__device__ __forceinline__ uint32_t radix_key(float v) {
  uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
  return (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
}

__device__ __forceinline__ uint64_t composite(float v, int64_t column) {
  return ((uint64_t)radix_key(v) << 32) | (uint64_t)(~(uint32_t)column);
}

struct Shared {
  uint32_t hist[kBins];
  uint64_t sel[kMaxK];
  uint64_t buf[kRefineCap];
  uint32_t wave_sums[kThreads / 64];
  uint32_t n_sel;
  uint32_t n_buf;
  uint32_t digit;
  uint32_t above;
  uint32_t bucket;
};

// Find the bucket d holding the `remaining`-th largest element: the suffix
// count above d is < remaining <= suffix count including d. Thread t owns
// bins 2t and 2t+1.
__device__ void find_bucket(Shared& sh, uint32_t remaining) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t h0 = sh.hist[2 * tid];
  const uint32_t h1 = sh.hist[2 * tid + 1];
  uint32_t local = h0 + h1;
  // inclusive prefix over threads
  uint32_t incl = local;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) sh.wave_sums[wave] = incl;
  __syncthreads();
  uint32_t before = 0, total = 0;
  for (int i = 0; i < kThreads / 64; ++i) {
    const uint32_t s = sh.wave_sums[i];
    if (i < wave) before += s;
    total += s;
  }
  incl += before;
  // Suffix counts: elements in bins strictly above this thread's pair.
  const uint32_t above_pair = total - incl;
  const uint32_t s1 = above_pair + h1;  // count at or above bin 2t+1
  const uint32_t s0 = s1 + h0;          // count at or above bin 2t
  if (h1 && above_pair < remaining && s1 >= remaining) {
    sh.digit = 2 * tid + 1;
    sh.above = above_pair;
    sh.bucket = h1;
  } else if (h0 && s1 < remaining && s0 >= remaining) {
    sh.digit = 2 * tid;
    sh.above = s1;
    sh.bucket = h0;
  }
  __syncthreads();
}

__device__ __forceinline__ void clear_hist(Shared& sh) {
  for (int i = threadIdx.x; i < kBins; i += kThreads) sh.hist[i] = 0;
}

template <typename F>
__device__ __forceinline__ void for_each_element(const float* row, int64_t cols, bool vec, F&& f) {
  if (vec) {
    const int64_t nvec = cols >> 2;
    const float4* row4 = reinterpret_cast<const float4*>(row);
    for (int64_t i = threadIdx.x; i < nvec; i += kThreads) {
      const float4 v = row4[i];
      f(v.x, 4 * i);
      f(v.y, 4 * i + 1);
      f(v.z, 4 * i + 2);
      f(v.w, 4 * i + 3);
    }
    for (int64_t i = 4 * nvec + threadIdx.x; i < cols; i += kThreads) f(row[i], i);
  } else {
    for (int64_t i = threadIdx.x; i < cols; i += kThreads) f(row[i], i);
  }
}

__global__ __launch_bounds__(kThreads, 1) void topk_rows(const float* __restrict__ scores,
                                                        int64_t cols, int64_t ld, int count,
                                                        float* __restrict__ values,
                                                        int32_t* __restrict__ ids,
                                                        int64_t out_ld) {
  __shared__ Shared sh;
  const int tid = threadIdx.x;
  const float* row = scores + (int64_t)blockIdx.x * ld;
  const bool vec = ((reinterpret_cast<uintptr_t>(row) & 15) == 0);

  if (tid == 0) {
    sh.n_sel = 0;
    sh.n_buf = 0;
  }
  if (count >= cols) {
    __syncthreads();
    for (int64_t i = tid; i < cols; i += kThreads) sh.sel[i] = composite(row[i], i);
  } else {
    // ---- level 0 histogram over the row
    clear_hist(sh);
    __syncthreads();
    for_each_element(row, cols, vec, [&](float v, int64_t) {
      atomicAdd(&sh.hist[radix_key(v) >> 21], 1u);
    });
    __syncthreads();
    uint32_t remaining = (uint32_t)count;
    find_bucket(sh, remaining);
    uint64_t prefix = (uint64_t)sh.digit << kShift[0];
    int shift = kShift[0];
    remaining -= sh.above;
    bool resolved = sh.bucket == remaining;
    const bool in_lds = !resolved && sh.bucket <= (uint32_t)kRefineCap;
    __syncthreads();

    if (in_lds) {
      const uint64_t d0 = prefix >> shift;
      for_each_element(row, cols, vec, [&](float v, int64_t i) {
        const uint64_t key = composite(v, i);
        const uint64_t d = key >> 53;
        if (d > d0) {
          const uint32_t slot = atomicAdd(&sh.n_sel, 1u);
          if (slot < kMaxK) sh.sel[slot] = key;
        } else if (d == d0) {
          const uint32_t slot = atomicAdd(&sh.n_buf, 1u);
          if (slot < kRefineCap) sh.buf[slot] = key;
        }
      });
      __syncthreads();
      const uint32_t nbuf = sh.n_buf < kRefineCap ? sh.n_buf : kRefineCap;
      for (int level = 1; level < kLevels && !resolved; ++level) {
        clear_hist(sh);
        __syncthreads();
        const int s = kShift[level];
        const uint64_t mask = (1ull << kWidth[level]) - 1;
        for (uint32_t i = tid; i < nbuf; i += kThreads) {
          const uint64_t key = sh.buf[i];
          if ((key >> shift) == (prefix >> shift)) atomicAdd(&sh.hist[(key >> s) & mask], 1u);
        }
        __syncthreads();
        find_bucket(sh, remaining);
        prefix |= (uint64_t)sh.digit << s;
        shift = s;
        remaining -= sh.above;
        resolved = sh.bucket == remaining;
        __syncthreads();
      }
      for (uint32_t i = tid; i < nbuf; i += kThreads) {
        const uint64_t key = sh.buf[i];
        if ((key >> shift) >= (prefix >> shift)) {
          const uint32_t slot = atomicAdd(&sh.n_sel, 1u);
          if (slot < kMaxK) sh.sel[slot] = key;
        }
      }
    } else {
      for (int level = 1; level < kLevels && !resolved; ++level) {
        clear_hist(sh);
        __syncthreads();
        const int s = kShift[level];
        const uint64_t mask = (1ull << kWidth[level]) - 1;
        const uint64_t want = prefix >> shift;
        const int cur = shift;
        for_each_element(row, cols, vec, [&](float v, int64_t i) {
          const uint64_t key = composite(v, i);
          if ((key >> cur) == want) atomicAdd(&sh.hist[(key >> s) & mask], 1u);
        });
        __syncthreads();
        find_bucket(sh, remaining);
        prefix |= (uint64_t)sh.digit << s;
        shift = s;
        remaining -= sh.above;
        resolved = sh.bucket == remaining;
        __syncthreads();
      }
      const uint64_t floor = prefix >> shift;
      const int cur = shift;
      for_each_element(row, cols, vec, [&](float v, int64_t i) {
        const uint64_t key = composite(v, i);
        if ((key >> cur) >= floor) {
          const uint32_t slot = atomicAdd(&sh.n_sel, 1u);
          if (slot < kMaxK) sh.sel[slot] = key;
        }
      });
    }
  }
  __syncthreads();

  // ---- bitonic sort of `count` keys, descending (padding keys are 0).
  int padded = 1;
  while (padded < count) padded <<= 1;
  for (int i = count + tid; i < padded; i += kThreads) sh.sel[i] = 0;
  __syncthreads();
  for (int size = 2; size <= padded; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < (padded >> 1); i += kThreads) {
        const int lo = 2 * stride * (i / stride) + (i % stride);
        const int hi = lo + stride;
        const uint64_t a = sh.sel[lo];
        const uint64_t b = sh.sel[hi];
        const bool descending = (lo & size) == 0;
        if (descending ? (a < b) : (a > b)) {
          sh.sel[lo] = b;
          sh.sel[hi] = a;
        }
      }
      __syncthreads();
    }
  }

  float* vout = values + (int64_t)blockIdx.x * out_ld;
  int32_t* iout = ids + (int64_t)blockIdx.x * out_ld;
  for (int i = tid; i < count; i += kThreads) {
    const uint64_t key = sh.sel[i];
    const uint32_t bits = key_bits((uint32_t)(key >> 32));
    vout[i] = __uint_as_float(bits);
    const bool finite = (bits & 0x7F800000u) != 0x7F800000u;
    iout[i] = finite ? (int32_t)(~(uint32_t)key) : -1;
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_topk_radix(const float* scores, int64_t rows, int64_t columns, int64_t ld,
                              int64_t k, float* values, int32_t* indices, int64_t out_ld,
                              hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(columns >= 1, "scores must have nonempty visible tokens");
  DSA_CHECK_ARG(k >= 1 && k <= kMaxK, "k must be an integer in [1, 2048]");
  DSA_CHECK_ARG(ld >= columns && rows >= 0, "invalid score layout");
  DSA_CHECK_ARG(columns < (int64_t)0x7FFFFFFF, "column count must fit int32");
  const int64_t count = k < columns ? k : columns;
  DSA_CHECK_ARG(out_ld >= count, "output row stride too small");
  if (rows == 0) return kOk;
  DSA_CHECK_ARG(scores && values && indices, "null pointer");
  DSA_CHECK_ARG(rows < 0x7FFFFFFF, "too many rows");
  hipLaunchKernelGGL(topk_rows, dim3((unsigned)rows), dim3(kThreads), 0, stream, scores, columns,
                     ld, (int)count, values, indices, out_ld);
  DSA_CHECK_LAUNCH("exact top-k");
  return kOk;
}
