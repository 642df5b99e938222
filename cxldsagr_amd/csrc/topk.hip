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
// 1. the row (or its half, below) is read once into registers as radix
//    keys; each thread's two largest keys bound the count-th largest from
//    below, and only keys at or above that bound are histogrammed on their
//    top 11 bits;
// 2. a pass over the registers sends keys above the threshold bucket to the
//    selected set in LDS and keys in the bucket to an LDS refine buffer;
// 3. the remaining digits (11/10/11/11/10 bits) are resolved on the LDS
//    buffer; a bucket too large for LDS (huge ties, e.g. masked rows) falls
//    back to further histogram passes over the row;
// 4. the <= 2048 selected keys are sorted: a counting sort into 2048 linear
//    buckets over their own key range plus in-bucket ranks, or, when a
//    bucket holds more than 32 keys, a bitonic network (two keys per thread;
//    partners within a wave exchanged with DPP / row-swap lane moves, only
//    strides of 128 and more through LDS); values and indices are decoded
//    from the keys.
//
// One 1024-thread work-group per row, or, for rows of 8192 columns and more
// through dsa_topk_radix_split, one per half-row: each half selects and
// sorts its own top min(count, half) keys into a workspace and a second
// launch merges the two sorted lists of every row (merge path), so Q rows
// occupy 2Q compute units.
#include <mutex>

#include "dsa_common.h"
#include "logits_core.h"
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

constexpr int kSubHists = 4;  // histogram copies (by wave % 4) against atomic contention

struct Shared {
  uint32_t hist[kSubHists][kBins];
  uint64_t sel[kMaxK];
  uint64_t buf[kRefineCap];
  uint32_t wave_sums[kThreads / 64];
  uint64_t wave_max[kThreads / 64];
  uint64_t wave_min[kThreads / 64];
  uint32_t sort_fallback;
  uint32_t n_sel;
  uint32_t n_buf;
  uint32_t digit;
  uint32_t above;
  uint32_t bucket;
  uint32_t total;
};

// Find the bucket d holding the `remaining`-th largest element: the suffix
// count above d is < remaining <= suffix count including d. Thread t owns
// bins 2t and 2t+1.
__device__ void find_bucket(Shared& sh, uint32_t remaining) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint32_t h0 = 0, h1 = 0;
#pragma unroll
  for (int c = 0; c < kSubHists; ++c) {
    h0 += sh.hist[c][2 * tid];
    h1 += sh.hist[c][2 * tid + 1];
  }
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
  if (tid == 0) sh.total = total;
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

// Slot allocation with one LDS atomic per wave: lanes with `take` get
// consecutive slots of `counter` in lane order.
__device__ __forceinline__ uint32_t wave_slot(uint32_t* counter, bool take) {
  const uint64_t mask = __builtin_amdgcn_ballot_w64(take);
  if (mask == 0) return 0;
  const uint32_t lanes_below =
      __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
  const int leader = __builtin_ffsll((long long)mask) - 1;
  uint32_t base = 0;
  if ((int)(threadIdx.x & 63) == leader) base = atomicAdd(counter, (uint32_t)__builtin_popcountll(mask));
  return __builtin_amdgcn_readlane(base, leader) + lanes_below;
}

// Value of lane (lane ^ kM) for kM = 1 .. 32 with VALU-only lane moves:
// quad permutes (DPP quad_perm) for 1 and 2; for 4 and 8 a quad reversal
// (lane ^ 3) or row mirror (lane ^ 15) followed by a half-row mirror
// (lane ^ 7); for 16 and 32 the gfx950 row-swap permutes, whose result
// pair holds (even row, odd row) of each row pair.
template <int kM>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (kM == 1) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
  } else if constexpr (kM == 2) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
  } else if constexpr (kM == 4) {
    return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x1B, 0xF, 0xF, false), 0x141, 0xF, 0xF, false);
  } else if constexpr (kM == 8) {
    return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false), 0x141, 0xF, 0xF, false);
  } else if constexpr (kM == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? p[0] : p[1];
  } else {
    static_assert(kM == 32, "lane distance");
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? p[0] : p[1];
  }
}

template <int kM>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
  return ((uint64_t)lane_xor<kM>((uint32_t)(v >> 32)) << 32) | lane_xor<kM>((uint32_t)v);
}

__device__ __forceinline__ void clear_hist(Shared& sh) {
  for (int i = threadIdx.x; i < kSubHists * kBins; i += kThreads) (&sh.hist[0][0])[i] = 0;
}

__device__ __forceinline__ uint32_t* my_hist(Shared& sh) { return sh.hist[(threadIdx.x >> 6) % kSubHists]; }

// Counting sort of the unique keys sh.sel[0 .. count), descending: 2048
// linear buckets over the keys' own range [smallest, largest] (so equal
// values spread over their column bits), scatter, then place each key by its
// rank inside its bucket. Returns false, leaving sh.sel as it was, when a bucket holds
// more than kMaxBucket keys (the caller then runs the bitonic network).
constexpr uint32_t kMaxBucket = 32;
__device__ bool counting_sort(Shared& sh, int count) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint32_t* counts = sh.hist[0];
  uint32_t* start = sh.hist[1];
  uint32_t* cursor = sh.hist[2];
  for (int i = tid; i < kBins; i += kThreads) counts[i] = 0;
  if (tid == 0) sh.sort_fallback = 0;
  uint64_t kmax = 0, kmin = ~0ull;
  for (int i = tid; i < count; i += kThreads) {
    const uint64_t key = sh.sel[i];
    kmax = key > kmax ? key : kmax;
    kmin = key < kmin ? key : kmin;
  }
  auto reduce = [&](auto m_tag) {
    constexpr int kM = decltype(m_tag)::value;
    const uint64_t a = lane_xor64<kM>(kmax), b = lane_xor64<kM>(kmin);
    kmax = a > kmax ? a : kmax;
    kmin = b < kmin ? b : kmin;
  };
  reduce(std::integral_constant<int, 1>{});
  reduce(std::integral_constant<int, 2>{});
  reduce(std::integral_constant<int, 4>{});
  reduce(std::integral_constant<int, 8>{});
  reduce(std::integral_constant<int, 16>{});
  reduce(std::integral_constant<int, 32>{});
  if (lane == 0) {
    sh.wave_max[wave] = kmax;
    sh.wave_min[wave] = kmin;
  }
  __syncthreads();
  kmax = sh.wave_max[0];
  kmin = sh.wave_min[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) {
    kmax = sh.wave_max[w] > kmax ? sh.wave_max[w] : kmax;
    kmin = sh.wave_min[w] < kmin ? sh.wave_min[w] : kmin;
  }
  // Linear buckets over [kmin, kmax]: the key distance from kmin, scaled to
  // 11 bits (monotone in the key).
  const uint64_t span = kmax - kmin;
  const int bits = span == 0 ? 0 : 64 - __builtin_clzll(span);
  const int shift = bits > 11 ? bits - 11 : 0;
  auto digit = [kmin, shift](uint64_t key) -> uint32_t { return (uint32_t)((key - kmin) >> shift); };
  for (int i = tid; i < count; i += kThreads) atomicAdd(&counts[digit(sh.sel[i])], 1u);
  __syncthreads();
  // Bucket starts in descending digit order; thread t owns bins 2t, 2t + 1.
  const uint32_t h0 = counts[2 * tid], h1 = counts[2 * tid + 1];
  uint32_t incl = h0 + h1;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) sh.wave_sums[wave] = incl;
  if (h0 > kMaxBucket || h1 > kMaxBucket) sh.sort_fallback = 1;
  __syncthreads();
  uint32_t before = 0;
  for (int w = 0; w < wave; ++w) before += sh.wave_sums[w];
  const uint32_t above_pair = (uint32_t)count - (incl + before);
  start[2 * tid + 1] = above_pair;
  cursor[2 * tid + 1] = above_pair;
  start[2 * tid] = above_pair + h1;
  cursor[2 * tid] = above_pair + h1;
  __syncthreads();
  if (sh.sort_fallback) return false;
  for (int i = tid; i < count; i += kThreads) {
    const uint64_t key = sh.sel[i];
    sh.buf[atomicAdd(&cursor[digit(key)], 1u)] = key;
  }
  __syncthreads();
  for (int i = tid; i < count; i += kThreads) {
    const uint64_t key = sh.buf[i];
    const uint32_t d = digit(key);
    const uint32_t b0 = start[d], n = counts[d];
    uint32_t rank = 0;
    for (uint32_t j = b0; j < b0 + n; ++j) rank += sh.buf[j] > key ? 1u : 0u;
    sh.sel[b0 + rank] = key;
  }
  __syncthreads();
  return true;
}

// Sorts the `count` unique keys sh.sel[0 .. count) in place, descending:
// counting sort, or when a bucket is crowded, a bitonic network (padding
// keys are 0). Thread t holds positions 2t and 2t + 1 in registers;
// partners at stride 1 are in the same thread, strides 2..64 in the same
// wave, strides >= 128 in LDS. Ends with a barrier.
__device__ __forceinline__ void sort_selected(Shared& sh, int count) {
  const int tid = threadIdx.x;
  if (!counting_sort(sh, count)) {
    int padded = 2;
    while (padded < count) padded <<= 1;
    for (int i = count + tid; i < padded; i += kThreads) sh.sel[i] = 0;
    __syncthreads();
    const bool active = 2 * tid < padded;
    uint64_t x0 = active ? sh.sel[2 * tid] : 0;
    uint64_t x1 = active ? sh.sel[2 * tid + 1] : 0;
    const int p0 = 2 * tid;
    const int lane = tid & 63;
    // Compare-exchange of a pair (lo at the lower position): the larger key
    // goes first inside descending blocks.
    auto order = [](uint64_t& lo, uint64_t& hi, bool descending) {
      const bool swap = (lo < hi) == descending;
      const uint64_t a = lo, b = hi;
      lo = swap ? b : a;
      hi = swap ? a : b;
    };
    // Strides 2..16: partner lane ^ kM (kM = stride / 2), fetched by DPP; the
    // lane keeps the larger key iff it holds the lower position of a
    // descending block (or the upper of an ascending one).
    auto exchange_dpp = [&](auto m_tag, int size) {
      constexpr int kM = decltype(m_tag)::value;
      const bool desc = (p0 & size) == 0;
      const bool keep_max = ((lane & kM) == 0) == desc;
      const uint64_t y0 = lane_xor64<kM>(x0);
      const uint64_t y1 = lane_xor64<kM>(x1);
      x0 = ((x0 < y0) == keep_max) ? y0 : x0;
      x1 = ((x1 < y1) == keep_max) ? y1 : x1;
    };
    // Strides 32 and 64 (lane ^ 16, lane ^ 32): one row-swap permute of (x0,
    // x1) leaves every lane holding a whole pair - lanes with the distance bit
    // clear get x0 of lanes l and l + kM, the others x1 of lanes l - kM and l -
    // so the exchange happens in-lane and a second permute restores the layout.
    auto exchange_swap = [&](auto m_tag, int size) {
      constexpr int kM = decltype(m_tag)::value;
      auto swap32 = [](uint32_t& a, uint32_t& b) {
        const auto r = kM == 16 ? __builtin_amdgcn_permlane16_swap(a, b, false, false)
                                : __builtin_amdgcn_permlane32_swap(a, b, false, false);
        a = r[0];
        b = r[1];
      };
      uint32_t a_lo = (uint32_t)x0, a_hi = (uint32_t)(x0 >> 32);
      uint32_t b_lo = (uint32_t)x1, b_hi = (uint32_t)(x1 >> 32);
      swap32(a_lo, b_lo);
      swap32(a_hi, b_hi);
      // The pair's lower position: 2l (x0 of lane l) or 2 (l - kM) + 1.
      const int first = (lane & kM) ? 2 * ((tid & ~63) + lane - kM) + 1 : p0;
      uint64_t lo = ((uint64_t)a_hi << 32) | a_lo;
      uint64_t hi = ((uint64_t)b_hi << 32) | b_lo;
      order(lo, hi, (first & size) == 0);
      a_lo = (uint32_t)lo;
      a_hi = (uint32_t)(lo >> 32);
      b_lo = (uint32_t)hi;
      b_hi = (uint32_t)(hi >> 32);
      swap32(a_lo, b_lo);
      swap32(a_hi, b_hi);
      x0 = ((uint64_t)a_hi << 32) | a_lo;
      x1 = ((uint64_t)b_hi << 32) | b_lo;
    };
    for (int size = 2; size <= padded; size <<= 1) {
      // Strides 128 .. size / 2 through LDS.
      for (int stride = size >> 1; stride >= 128; stride >>= 1) {
        const bool desc = (p0 & size) == 0;
        if (active) {
          sh.sel[p0] = x0;
          sh.sel[p0 + 1] = x1;
        }
        __syncthreads();
        const uint64_t y0 = active ? sh.sel[p0 ^ stride] : 0;
        const uint64_t y1 = active ? sh.sel[(p0 + 1) ^ stride] : 0;
        const bool keep_max = ((p0 & stride) == 0) == desc;
        x0 = ((x0 < y0) == keep_max) ? y0 : x0;
        x1 = ((x1 < y1) == keep_max) ? y1 : x1;
        __syncthreads();
      }
      if (size >= 128) exchange_swap(std::integral_constant<int, 32>{}, size);
      if (size >= 64) exchange_swap(std::integral_constant<int, 16>{}, size);
      if (size >= 32) exchange_dpp(std::integral_constant<int, 8>{}, size);
      if (size >= 16) exchange_dpp(std::integral_constant<int, 4>{}, size);
      if (size >= 8) exchange_dpp(std::integral_constant<int, 2>{}, size);
      if (size >= 4) exchange_dpp(std::integral_constant<int, 1>{}, size);
      order(x0, x1, (p0 & size) == 0);
    }
    if (active) {
      sh.sel[p0] = x0;
      sh.sel[p0 + 1] = x1;
    }
    __syncthreads();
  }
}

// Calls f(value, column) for every element of the row, each thread with four
// 16-byte loads in flight.
template <typename F>
__device__ __forceinline__ void for_each_element(const float* row, int64_t cols, bool vec, F&& f) {
  if (vec) {
    const int64_t nvec = cols >> 2;
    const float4* row4 = reinterpret_cast<const float4*>(row);
    constexpr int kDepth = 4;
    int64_t i = threadIdx.x;
    for (; i + (kDepth - 1) * kThreads < nvec; i += kDepth * kThreads) {
      float4 v[kDepth];
#pragma unroll
      for (int d = 0; d < kDepth; ++d) v[d] = row4[i + d * kThreads];
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int64_t c = 4 * (i + d * kThreads);
        f(v[d].x, c);
        f(v[d].y, c + 1);
        f(v[d].z, c + 2);
        f(v[d].w, c + 3);
      }
    }
    for (; i < nvec; i += kThreads) {
      const float4 v = row4[i];
      f(v.x, 4 * i);
      f(v.y, 4 * i + 1);
      f(v.z, 4 * i + 2);
      f(v.w, 4 * i + 3);
    }
    for (int64_t j = 4 * nvec + threadIdx.x; j < cols; j += kThreads) f(row[j], j);
  } else {
    for (int64_t j = threadIdx.x; j < cols; j += kThreads) f(row[j], j);
  }
}

// The keys of the level-0 bucket (the `prefix >> shift` digit) still to be
// split, `remaining` of them wanted: with the bucket's keys in sh.buf[0 ..
// nbuf), further digits (11/10/11/11/10 bits) narrow it to exactly
// `remaining` keys, which are appended to sh.sel after its sh.n_sel keys.
__device__ __forceinline__ void refine_buffer(Shared& sh, uint64_t prefix, int shift, uint32_t remaining,
                              bool resolved, uint32_t nbuf) {
  const int tid = threadIdx.x;
  for (int level = 1; level < kLevels && !resolved; ++level) {
    clear_hist(sh);
    __syncthreads();
    const int s = kShift[level];
    const uint64_t mask = (1ull << kWidth[level]) - 1;
    for (uint32_t i = tid; i < nbuf; i += kThreads) {
      const uint64_t key = sh.buf[i];
      if ((key >> shift) == (prefix >> shift)) atomicAdd(&my_hist(sh)[(key >> s) & mask], 1u);
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
    const bool take = (key >> shift) >= (prefix >> shift);
    const uint32_t slot = wave_slot(&sh.n_sel, take);
    if (take && slot < kMaxK) sh.sel[slot] = key;
  }
}

// The same when the bucket is too large for LDS: each further digit is
// histogrammed over the row itself, and a last pass over the row appends
// every key at or above the final prefix (all `count` of them, so sh.sel
// starts empty).
__device__ __forceinline__ void refine_from_row(Shared& sh, const float* row, int64_t cols, bool vec, uint64_t prefix,
                                int shift, uint32_t remaining, bool resolved) {
  for (int level = 1; level < kLevels && !resolved; ++level) {
    clear_hist(sh);
    __syncthreads();
    const int s = kShift[level];
    const uint64_t mask = (1ull << kWidth[level]) - 1;
    const uint64_t want = prefix >> shift;
    const int cur = shift;
    for_each_element(row, cols, vec, [&](float v, int64_t i) {
      const uint64_t key = composite(v, i);
      if ((key >> cur) == want) atomicAdd(&my_hist(sh)[(key >> s) & mask], 1u);
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
    const bool take = (key >> cur) >= floor;
    const uint32_t slot = wave_slot(&sh.n_sel, take);
    if (take && slot < kMaxK) sh.sel[slot] = key;
  });
}

// Row elements in batches: each thread gets kBatch elements per call of f
// (values, columns, validity), loaded as kBatch / 4 float4 in flight, with
// every lane active in every call (invalid slots past the row end).
constexpr int kBatch = 16;
template <typename F>
__device__ __forceinline__ void for_each_batch(const float* row, int64_t cols, bool vec, F&& f) {
  const int64_t nvec = (cols + 3) >> 2;
  constexpr int kVec = kBatch / 4;
  for (int64_t base = 0; base < nvec; base += (int64_t)kVec * kThreads) {
    float v[kBatch];
    int64_t c[kVec];
#pragma unroll
    for (int d = 0; d < kVec; ++d) {
      const int64_t i = base + (int64_t)d * kThreads + threadIdx.x;
      c[d] = 4 * i;
      if (vec && 4 * i + 3 < cols) {
        const float4 x = reinterpret_cast<const float4*>(row)[i];
        v[4 * d] = x.x;
        v[4 * d + 1] = x.y;
        v[4 * d + 2] = x.z;
        v[4 * d + 3] = x.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * d + e] = 4 * i + e < cols ? row[4 * i + e] : 0.0f;
      }
    }
    f(v, c);
  }
}

// A row of up to kResident * kThreads elements is read from memory once and
// kept in registers (thread t: float4 slots d * kThreads + t) for both the
// histogram and the selection pass.
// Register capacities: 17 float4 per thread (69,632 columns) for whole rows,
// 9 (36,864) for the halves of split rows, so a thread walks only slots that
// can hold row elements.
constexpr int kResidentVecLarge = 17;
constexpr int kResidentVecSmall = 9;
constexpr int64_t resident_cols(int vecs) { return 4 * (int64_t)vecs * kThreads; }

template <int kResidentVec>
struct Resident {
  float v[4 * kResidentVec];
  __device__ __forceinline__ void load(const float* row, int64_t cols) {
#pragma unroll
    for (int d = 0; d < kResidentVec; ++d) {
      const int64_t i = (int64_t)d * kThreads + threadIdx.x;
      if (4 * i + 3 < cols) {
        const float4 x = reinterpret_cast<const float4*>(row)[i];
        v[4 * d] = x.x;
        v[4 * d + 1] = x.y;
        v[4 * d + 2] = x.z;
        v[4 * d + 3] = x.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * d + e] = 4 * i + e < cols ? row[4 * i + e] : 0.0f;
      }
    }
  }
  template <typename F>
  __device__ __forceinline__ void for_each(int64_t cols, F&& f) const {
#pragma unroll
    for (int d = 0; d < kResidentVec; ++d) {
      const int64_t c = 4 * ((int64_t)d * kThreads + threadIdx.x);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < cols) f(v[4 * d + e], c + e);
    }
  }
  // Batches of 16 values (4 float4 slots) in the for_each_batch format; slots
  // past kResidentVec get columns past the row end.
  template <typename F>
  __device__ __forceinline__ void for_each_batch(int64_t cols, F&& f) const {
#pragma unroll
    for (int b = 0; b < (kResidentVec + 3) / 4; ++b) {
      float bv[16];
      int64_t bc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = 4 * b + q;
        bc[q] = d < kResidentVec ? 4 * ((int64_t)d * kThreads + threadIdx.x) : cols;
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[4 * q + e] = d < kResidentVec ? v[4 * d + e] : 0.0f;
      }
      f(bv, bc);
    }
  }
};

// The work-group selects and sorts the top min(count, columns of its part)
// keys of row r's part `part` of `parts`. With one part that is the answer.
// With two (columns split at a multiple of 4 near the middle), each part
// stores its sorted keys in the workspace and topk_merge, launched next on
// the same stream, merges them.
template <int kResidentVec>
__device__ __forceinline__ void select_row(Shared& sh, const float* __restrict__ scores, int64_t all_cols,
                           int64_t ld, int total_count, float* __restrict__ values,
                           int32_t* __restrict__ ids, int64_t out_ld, uint64_t* ws_keys,
                           int64_t r, int part, int parts) {
  const int tid = threadIdx.x;
  const int64_t part_cols = parts == 1 ? all_cols : ((((all_cols + 1) >> 1) + 3) & ~(int64_t)3);
  const int64_t col0 = part * part_cols;
  const int64_t cols = part_cols < all_cols - col0 ? part_cols : all_cols - col0;
  const int count = total_count < cols ? total_count : (int)cols;
  const float* row = scores + r * ld + col0;
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
    const bool resident = vec && cols <= resident_cols(kResidentVec);
    Resident<kResidentVec> res;
    uint32_t floor_key = 0;  // radix keys below it cannot be among the top `count`
    // Resident slots e < n_valid hold row elements (columns grow with e).
    int n_valid = 0;
    if (resident) {
      res.load(row, cols);
#pragma unroll
      for (int d = 0; d < kResidentVec; ++d) {
        const int32_t left = (int32_t)cols - 4 * (d * kThreads + tid);
        n_valid += left <= 0 ? 0 : (left >= 4 ? 4 : left);
      }
      // Values -> radix keys in place, and each thread's two largest keys.
      // The 2048 >= count keys so found are a subset of the row, so their
      // minimum is at most the count-th largest key: every key below it can
      // be left out of the search (typically ~85-95 % of the row).
      uint32_t t1 = 0, t2 = 0;
#pragma unroll
      for (int e = 0; e < 4 * kResidentVec; ++e) {
        const uint32_t r = e < n_valid ? radix_key(res.v[e]) : 0u;
        res.v[e] = __uint_as_float(r);
        t2 = max(t2, min(t1, r));
        t1 = max(t1, r);
      }
      t2 = min(t2, lane_xor<1>(t2));
      t2 = min(t2, lane_xor<2>(t2));
      t2 = min(t2, lane_xor<4>(t2));
      t2 = min(t2, lane_xor<8>(t2));
      t2 = min(t2, lane_xor<16>(t2));
      t2 = min(t2, lane_xor<32>(t2));
      if ((tid & 63) == 0) sh.wave_sums[tid >> 6] = t2;
    }
    clear_hist(sh);
    __syncthreads();
    auto count_top = [&](float v, int64_t) { atomicAdd(&my_hist(sh)[radix_key(v) >> 21], 1u); };
    if (resident) {
      floor_key = sh.wave_sums[0];
#pragma unroll
      for (int w = 1; w < kThreads / 64; ++w) floor_key = min(floor_key, sh.wave_sums[w]);
      uint32_t* hist = my_hist(sh);
#pragma unroll
      for (int e = 0; e < 4 * kResidentVec; ++e) {
        const uint32_t r = __float_as_uint(res.v[e]);
        if (e < n_valid && r >= floor_key) atomicAdd(&hist[r >> 21], 1u);
      }
    } else {
      for_each_element(row, cols, vec, count_top);
    }
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
      const uint32_t d0_32 = (uint32_t)d0;
      const uint32_t lane = threadIdx.x & 63;
      auto select_batch = [&](const float (&v)[kBatch], const int64_t (&c)[kBatch / 4]) {
        // Per-lane counts of selected / candidate elements, their exclusive
        // prefix over the wave from 5 bit-plane ballots (counts <= 16), and
        // one LDS atomic per list per batch.
        uint32_t dig[kBatch];
        uint32_t cnt_sel = 0, cnt_buf = 0;
#pragma unroll
        for (int e = 0; e < kBatch; ++e) {
          const bool ok = (int32_t)(c[e / 4] + (e % 4)) < (int32_t)cols;
          dig[e] = ok ? radix_key(v[e]) >> 21 : 0xFFFFu;  // 0xFFFF: past the row end
          cnt_sel += (dig[e] > d0_32 && dig[e] != 0xFFFFu) ? 1u : 0u;
          cnt_buf += dig[e] == d0_32 ? 1u : 0u;
        }
        uint32_t pre_sel = 0, pre_buf = 0, tot_sel = 0, tot_buf = 0;
#pragma unroll
        for (int bit = 0; bit < 5; ++bit) {
          const uint64_t ms = __builtin_amdgcn_ballot_w64((cnt_sel >> bit) & 1u);
          const uint64_t mb = __builtin_amdgcn_ballot_w64((cnt_buf >> bit) & 1u);
          pre_sel += __builtin_amdgcn_mbcnt_hi((uint32_t)(ms >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ms, 0)) << bit;
          pre_buf += __builtin_amdgcn_mbcnt_hi((uint32_t)(mb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mb, 0)) << bit;
          tot_sel += (uint32_t)__builtin_popcountll(ms) << bit;
          tot_buf += (uint32_t)__builtin_popcountll(mb) << bit;
        }
        if (tot_sel + tot_buf == 0) return;
        uint32_t base_sel = 0, base_buf = 0;
        if (lane == 0) {
          if (tot_sel) base_sel = atomicAdd(&sh.n_sel, tot_sel);
          if (tot_buf) base_buf = atomicAdd(&sh.n_buf, tot_buf);
        }
        uint32_t at_sel = __builtin_amdgcn_readfirstlane(base_sel) + pre_sel;
        uint32_t at_buf = __builtin_amdgcn_readfirstlane(base_buf) + pre_buf;
#pragma unroll
        for (int e = 0; e < kBatch; ++e) {
          if (dig[e] == 0xFFFFu) continue;
          if (dig[e] > d0_32) {
            if (at_sel < kMaxK) sh.sel[at_sel] = composite(v[e], c[e / 4] + (e % 4));
            ++at_sel;
          } else if (dig[e] == d0_32) {
            if (at_buf < kRefineCap) sh.buf[at_buf] = composite(v[e], c[e / 4] + (e % 4));
            ++at_buf;
          }
        }
      };
      if (resident) {
        // Survivor masks first (bit e % 32 of word e / 32 for resident value
        // e, column 4 ((e / 4) kThreads + tid) + e % 4), then one pass over
        // the set bits only: survivors are a few percent of the row.
        constexpr int kValues = 4 * kResidentVec;
        constexpr int kWords = (kValues + 31) / 32;
        uint32_t m_sel[kWords], m_buf[kWords];
#pragma unroll
        for (int h = 0; h < kWords; ++h) {
          m_sel[h] = 0;
          m_buf[h] = 0;
        }
#pragma unroll
        for (int e = 0; e < kValues; ++e) {
          const uint32_t r = __float_as_uint(res.v[e]);  // radix key
          const uint32_t dig = r >> 21;
          const bool ok = e < n_valid;
          m_sel[e >> 5] |= (ok && dig > d0_32) ? 1u << (e & 31) : 0u;
          // Only keys the histogram counted (>= floor_key) enter the refinement.
          m_buf[e >> 5] |= (ok && dig == d0_32 && r >= floor_key) ? 1u << (e & 31) : 0u;
        }
        uint32_t cnt_sel = 0, cnt_buf = 0;
#pragma unroll
        for (int h = 0; h < kWords; ++h) {
          cnt_sel += (uint32_t)__builtin_popcount(m_sel[h]);
          cnt_buf += (uint32_t)__builtin_popcount(m_buf[h]);
        }
        // Exclusive prefix over the wave from bit-plane ballots (counts <= 68).
        uint32_t pre_sel = 0, pre_buf = 0, tot_sel = 0, tot_buf = 0;
#pragma unroll 1
        for (int bit = 0; bit < 7; ++bit) {
          const uint64_t ms = __builtin_amdgcn_ballot_w64((cnt_sel >> bit) & 1u);
          const uint64_t mb = __builtin_amdgcn_ballot_w64((cnt_buf >> bit) & 1u);
          pre_sel += __builtin_amdgcn_mbcnt_hi((uint32_t)(ms >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ms, 0)) << bit;
          pre_buf += __builtin_amdgcn_mbcnt_hi((uint32_t)(mb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mb, 0)) << bit;
          tot_sel += (uint32_t)__builtin_popcountll(ms) << bit;
          tot_buf += (uint32_t)__builtin_popcountll(mb) << bit;
        }
        uint32_t base_sel = 0, base_buf = 0;
        if (lane == 0) {
          if (tot_sel) base_sel = atomicAdd(&sh.n_sel, tot_sel);
          if (tot_buf) base_buf = atomicAdd(&sh.n_buf, tot_buf);
        }
        uint32_t at_sel = __builtin_amdgcn_readfirstlane(base_sel) + pre_sel;
        uint32_t at_buf = __builtin_amdgcn_readfirstlane(base_buf) + pre_buf;
        // Columns into the lists; the keys follow from the row (in L2).
#pragma unroll
        for (int h = 0; h < kWords; ++h) {
          uint32_t m = m_sel[h] | m_buf[h];
          while (m) {
            const int e = __builtin_ctz(m);
            m &= m - 1;
            const int idx = 32 * h + e;
            const uint32_t col = 4 * ((uint32_t)(idx >> 2) * kThreads + (uint32_t)tid) + (uint32_t)(idx & 3);
            if ((m_sel[h] >> e) & 1u) {
              if (at_sel < kMaxK) sh.sel[at_sel] = col;
              ++at_sel;
            } else {
              if (at_buf < kRefineCap) sh.buf[at_buf] = col;
              ++at_buf;
            }
          }
        }
        __syncthreads();
        const uint32_t ns = sh.n_sel < kMaxK ? sh.n_sel : kMaxK;
        const uint32_t nb = sh.n_buf < kRefineCap ? sh.n_buf : kRefineCap;
        for (uint32_t i = tid; i < ns + nb; i += kThreads) {
          uint64_t* slot = i < ns ? &sh.sel[i] : &sh.buf[i - ns];
          const uint32_t col = (uint32_t)*slot;
          *slot = composite(row[col], col);
        }
      } else {
        for_each_batch(row, cols, vec, select_batch);
      }
      __syncthreads();
      const uint32_t nbuf = sh.n_buf < kRefineCap ? sh.n_buf : kRefineCap;
      refine_buffer(sh, prefix, shift, remaining, resolved, nbuf);
    } else {
      refine_from_row(sh, row, cols, vec, prefix, shift, remaining, resolved);
    }
  }
  __syncthreads();

  sort_selected(sh, count);

  float* vout = values + r * out_ld;
  int32_t* iout = ids + r * out_ld;
  auto emit = [&](int i, uint64_t key) {
    const uint32_t bits = key_bits((uint32_t)(key >> 32));
    vout[i] = __uint_as_float(bits);
    const bool finite = (bits & 0x7F800000u) != 0x7F800000u;
    iout[i] = finite ? (int32_t)(~(uint32_t)key) : -1;
  };
  if (parts == 1) {
    for (int i = tid; i < count; i += kThreads) emit(i, sh.sel[i]);
    return;
  }

  // ---- two parts: this part's sorted list (row-global columns) goes to the
  // workspace; topk_merge combines the two lists of each row.
  uint64_t* mine = ws_keys + (r * 2 + part) * kMaxK;
  for (int i = tid; i < count; i += kThreads) {
    const uint64_t key = sh.sel[i];
    const uint32_t col = ~(uint32_t)key + (uint32_t)col0;
    mine[i] = (key & 0xFFFFFFFF00000000ull) | (uint64_t)(~col);
  }
}

// Work-group (r, h) of a grid (rows, parts): select_row for row r, part h.
template <int kResidentVec>
__global__ __launch_bounds__(kThreads, 1) void topk_rows(const float* __restrict__ scores,
                                                        int64_t all_cols, int64_t ld, int total_count,
                                                        float* __restrict__ values,
                                                        int32_t* __restrict__ ids,
                                                        int64_t out_ld, uint64_t* ws_keys) {
  __shared__ Shared sh;
  select_row<kResidentVec>(sh, scores, all_cols, ld, total_count, values, ids, out_ld, ws_keys,
                           blockIdx.x, blockIdx.y, gridDim.y);
}

// Merge path over the two descending key lists of a row (keys are unique):
// thread t emits outputs 2t and 2t + 1 of the top `count`.
__global__ __launch_bounds__(kThreads, 1) void topk_merge(const uint64_t* __restrict__ ws_keys,
                                                         int64_t all_cols, int count,
                                                         float* __restrict__ values,
                                                         int32_t* __restrict__ ids, int64_t out_ld) {
  __shared__ uint64_t A[kMaxK];
  __shared__ uint64_t B[kMaxK];
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int64_t part_cols = (((all_cols + 1) >> 1) + 3) & ~(int64_t)3;
  const int n_a = count < part_cols ? count : (int)part_cols;
  const int64_t rest = all_cols - part_cols;
  const int n_b = count < rest ? count : (int)rest;
  const uint64_t* src = ws_keys + r * 2 * kMaxK;
  for (int i = tid; i < n_a; i += kThreads) A[i] = src[i];
  for (int i = tid; i < n_b; i += kThreads) B[i] = src[kMaxK + i];
  __syncthreads();
  float* vout = values + r * out_ld;
  int32_t* iout = ids + r * out_ld;
  const int p = 2 * tid;
  if (p >= count) return;
  int lo = p - n_b > 0 ? p - n_b : 0;
  int hi = p < n_a ? p : n_a;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (A[mid] > B[p - 1 - mid]) lo = mid + 1;
    else hi = mid;
  }
  int i = lo, j = p - lo;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (p + q < count) {
      const bool take_a = i < n_a && (j >= n_b || A[i] > B[j]);
      const uint64_t key = take_a ? A[i] : B[j];
      if (take_a) ++i;
      else ++j;
      const uint32_t bits = key_bits((uint32_t)(key >> 32));
      vout[p + q] = __uint_as_float(bits);
      const bool finite = (bits & 0x7F800000u) != 0x7F800000u;
      iout[p + q] = finite ? (int32_t)(~(uint32_t)key) : -1;
    }
  }
}


// ---- exact top-k from precomputed level-0 digit counts.
//
// Workspace of R rows (columns read in P parts by the selection launch):
//   counts    u32 [R][kBins]  digit counts (added by the caller, zeroed here)
//   threshold u32 [R][8]      {valid, digit, above, bucket, top digit}
//   fill      u32 [R]         candidates listed so far (zero on entry and exit)
//   lists     u64 [R][kListCap]  the row's keys at or above the threshold
//                                digit (composite keys), in no order
// Counts and fill are zero on entry and exit; the rest is written before it
// is read.
// Selection work-groups: wave 0 reads the row's counts while waves 1-15 read
// kSelectVec float4 per thread of the row part (34,560 columns).
constexpr int kSelectVec = 9;
constexpr int kSelectDataThreads = kThreads - 64;
constexpr int kListCap = kMaxK + kRefineCap;  // candidates a row may list
constexpr int kWaveCap = 1024;                // candidates a wave stages in LDS
constexpr uint32_t kOverflow = 0x40000000u;   // added to a row's fill by an overflowing part
constexpr int kSortCap = kListCap;  // candidates the one-pass counting sort takes
constexpr int kSortBins = 4096;     // its linear buckets
constexpr uint32_t kSortBucketMax = 128;  // keys per bucket it ranks by comparison
constexpr int kSortPerThread = kSortCap / kThreads;
// List slots per thread the candidate top-k loads before it knows the lists'
// lengths (the rest after): at configs 1+2 a key split lists ~140 keys for its
// 32 threads, i.e. ~4.4 slots per thread. Three cover most of the keys while
// the records load; more read slots past the lists' ends (5: 1.15x the
// launch's algorithmic bytes, 3: 1.09x, the same time).
constexpr int kSpecSlots = 3;
constexpr int kSortEager = 4;  // key slots per thread loaded before the row's count is known

struct DigitWorkspace {
  uint32_t* counts;
  uint32_t* threshold;
  uint32_t* fill;
  uint64_t* lists;
  int parts;
};

int64_t select_parts(int64_t columns) {
  const int64_t span = 4 * (int64_t)kSelectVec * kSelectDataThreads;
  return (columns + span - 1) / span;
}

int64_t digit_workspace_bytes(int64_t rows, int64_t columns) {
  (void)columns;
  const int64_t fill = (rows * 4 + 7) & ~(int64_t)7;
  return rows * ((int64_t)kBins * 4 + 32) + fill + rows * (int64_t)kListCap * 8;
}

DigitWorkspace digit_workspace(void* base, int64_t rows, int64_t columns) {
  DigitWorkspace ws;
  ws.parts = (int)select_parts(columns);
  ws.counts = static_cast<uint32_t*>(base);
  ws.threshold = ws.counts + rows * kBins;
  ws.fill = ws.threshold + rows * 8;
  ws.lists = reinterpret_cast<uint64_t*>(ws.fill + ((rows + 1) & ~(int64_t)1));
  return ws;
}

struct Threshold {
  uint32_t digit;   // level-0 digit whose bucket holds the count-th largest key
  uint32_t above;   // keys in higher digits (< count)
  uint32_t bucket;  // keys in that digit (above + bucket >= count)
  uint32_t top;     // highest digit with a key
  uint32_t total;   // sum of the counts
};

// The level-0 threshold of a row from its kBins digit counts, computed by
// one wave without barriers: lane l holds digits 32l .. 32l + 31.
__device__ __forceinline__ Threshold row_threshold(const uint32_t* __restrict__ row_counts,
                                                   uint32_t count) {
  const int lane = threadIdx.x & 63;
  uint32_t c[32];
  const uint4* src = reinterpret_cast<const uint4*>(row_counts + 32 * lane);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint4 x = src[q];
    c[4 * q] = x.x;
    c[4 * q + 1] = x.y;
    c[4 * q + 2] = x.z;
    c[4 * q + 3] = x.w;
  }
  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < 32; ++j) sum += c[j];
  // Keys in lanes >= this one (higher lanes hold higher digits).
  uint32_t incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_down(incl, d);
    if (lane + d < 64) incl += o;
  }
  Threshold t{0u, 0u, 0u, 0u, (uint32_t)__shfl(incl, 0)};
  const uint32_t above_lane = incl - sum;
  const bool mine = above_lane < count && incl >= count;
  uint32_t digit = 0, above = 0, bucket = 0, top = 0, acc = above_lane;
#pragma unroll
  for (int j = 31; j >= 0; --j) {
    if (mine && acc < count && acc + c[j] >= count) {
      digit = 32 * lane + j;
      above = acc;
      bucket = c[j];
    }
    if (top == 0 && c[j]) top = 32 * lane + j + 1;  // + 1: 0 means none yet
    acc += c[j];
  }
  const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
  if (m) {
    const int leader = __builtin_ffsll((long long)m) - 1;
    t.digit = __builtin_amdgcn_readlane(digit, leader);
    t.above = __builtin_amdgcn_readlane(above, leader);
    t.bucket = __builtin_amdgcn_readlane(bucket, leader);
  }
  const uint64_t nonempty = __builtin_amdgcn_ballot_w64(sum != 0);
  if (nonempty) {
    const int highest = 63 - __builtin_clzll(nonempty);
    t.top = __builtin_amdgcn_readlane(top, highest) - 1;
  }
  return t;
}

// Exclusive prefix over the wave of per-lane counts below 64, and the total.
__device__ __forceinline__ uint32_t wave_prefix(uint32_t n, uint32_t* total) {
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < 6; ++bit) {
    const uint64_t m = __builtin_amdgcn_ballot_w64((n >> bit) & 1u);
    pre += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0)) << bit;
    tot += (uint32_t)__builtin_popcountll(m) << bit;
  }
  *total = tot;
  return pre;
}

// Exclusive prefix over the wave of any per-lane counts, and the total.
__device__ __forceinline__ uint32_t wave_prefix_any(uint32_t n, uint32_t* total) {
  const int lane = threadIdx.x & 63;
  uint32_t incl = n;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  *total = __shfl(incl, 63);
  return incl - n;
}

typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

struct SelectShared {
  uint32_t staged[kThreads / 64][2][kWaveCap + 1];  // [wave][score bits, column code][slot]
  uint32_t wave_count[kThreads / 64];
  uint32_t digit, total, listed;
};

// Work-group (r, p) of a grid (rows, parts): reads part p of row r once and
// lists its candidates - keys at or above the row's threshold digit - when
// the row's candidates fit kListCap: each wave stages its own (score bits and
// column code) in LDS in column order (positions from ballots, no atomics;
// the radix keys are formed in the copy); one atomic on the row's
// fill then places the part's candidates in the row's list, where the waves
// copy them in whole lines. Part 0 also stores the row's threshold record.
__global__ __launch_bounds__(kThreads, 1) void topk_digit_select(const float* __restrict__ scores,
                                                                int64_t cols, int64_t ld, int count,
                                                                int64_t part_cols,
                                                                DigitWorkspace ws) {
  __shared__ SelectShared ss;
  __shared__ uint32_t list_base;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t r = blockIdx.x;
  const int part = blockIdx.y;
  const int64_t col0 = (int64_t)part * part_cols;
  const uint32_t n = (uint32_t)(part_cols < cols - col0 ? part_cols : cols - col0);
  const float* row = scores + r * ld + col0;
  const bool vec = (reinterpret_cast<uintptr_t>(row) & 15) == 0;
  // Slot e of data thread dt = tid - 64 (waves 1-15): column
  // 4 ((e / 4) kSelectDataThreads + dt) + e % 4 of the part.
  const int dt = tid - 64;
  auto column = [dt](int e) {
    return 4u * ((uint32_t)(e >> 2) * kSelectDataThreads + (uint32_t)dt) + (uint32_t)(e & 3);
  };
  uint32_t bits[4 * kSelectVec];
  if (wave == 0) {
    const Threshold t = row_threshold(ws.counts + r * kBins, (uint32_t)count);
    if (lane == 0) {
      ss.digit = t.digit;
      ss.total = t.total;
      ss.listed = t.above + t.bucket <= (uint32_t)kListCap;
      if (part == 0) {
        uint32_t* rec = ws.threshold + r * 8;
        rec[0] = t.total == (uint32_t)cols;
        rec[1] = t.digit;
        rec[2] = t.above;
        rec[3] = t.bucket;
        rec[4] = t.top;
      }
    }
#pragma unroll
    for (int e = 0; e < 4 * kSelectVec; ++e) bits[e] = 0;
  } else {
    // Raw buffer loads over the part's n columns: dwords past the end read
    // as 0 (the hardware's range check), so every load is unconditional and
    // the waits for them can follow the loads in order.
    const __amdgpu_buffer_rsrc_t part_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), (short)0, (int)(n * 4), 0x00020000);
    if (vec) {
#pragma unroll
      for (int d = 0; d < kSelectVec; ++d) {
        const v4u32 x = __builtin_amdgcn_raw_buffer_load_b128(part_rsrc, (int)(column(4 * d) * 4), 0, 0);
        bits[4 * d] = x.x;
        bits[4 * d + 1] = x.y;
        bits[4 * d + 2] = x.z;
        bits[4 * d + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4 * kSelectVec; ++e)
        bits[e] = __builtin_amdgcn_raw_buffer_load_b32(part_rsrc, (int)(column(e) * 4), 0, 0);
    }
  }
  __syncthreads();
  // Rows whose counts do not sum to the row, or whose candidates do not fit
  // the list, are selected by topk_digit_finish from their scores.
  if (ss.total != (uint32_t)cols || !ss.listed) return;
  const uint32_t d0 = ss.digit;
  const uint32_t floor_key = d0 << 21;
  // A non-negative threshold (d0 >= 1024) compares the raw bits as signed
  // integers: negative values are below it, non-negative ones order by bits.
  const bool nonnegative = d0 >= 1024;
  const int32_t floor_bits = (int32_t)((d0 - 1024) << 21);
  const uint32_t not_col0 = ~(uint32_t)col0;
  uint32_t(*staged)[kWaveCap + 1] = ss.staged[wave];
  const uint32_t col_base = not_col0 - 4u * (uint32_t)dt;  // not_col0 - column(e) = col_base - offset(e)
  uint32_t off = 0;  // wave-uniform
  // Staged entries hold the raw score bits; the copy below turns them into
  // radix keys (a fraction of the elements reach it).
  auto stage = [&](int e, bool hit) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
    // Slot kWaveCap takes every entry past the wave's capacity (a part with
    // such a wave is not listed).
    const uint32_t pos = min(__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, off)),
                             (uint32_t)kWaveCap);
    if (hit) {
      staged[0][pos] = bits[e];
      staged[1][pos] = col_base - (4u * (uint32_t)(e >> 2) * kSelectDataThreads + (uint32_t)(e & 3));
    }
    off += (uint32_t)__builtin_popcountll(m);
  };
  if (wave != 0) {  // wave 0 holds no keys
    if (nonnegative && d0 > 1024) {
      // Above +0.0: one signed compare per key, and the zeros read past the
      // part's end can never pass it.
#pragma unroll
      for (int e = 0; e < 4 * kSelectVec; ++e)
        stage(e, (int32_t)bits[e] >= floor_bits);
    } else {
#pragma unroll
      for (int e = 0; e < 4 * kSelectVec; ++e) {
        stage(e, radix_key(__uint_as_float(bits[e])) >= floor_key && column(e) < n);
      }
    }
  }
  if (lane == 0) ss.wave_count[wave] = off;
  __syncthreads();
  uint32_t before = 0, total = 0;
  bool overflow = false;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    const uint32_t cw = ss.wave_count[w];
    before += w < wave ? cw : 0u;
    total += cw;
    overflow |= cw > (uint32_t)kWaveCap;
  }
  if (tid == 0) list_base = atomicAdd(&ws.fill[r], overflow ? kOverflow : total);
  __syncthreads();
  const uint32_t base = list_base;
  // (The fill tells the finish. Compared without a sum that could wrap: a
  // fill that is not zero on entry - a workspace reused with another row
  // count - must not place the list anywhere but inside it.)
  if (overflow || base > (uint32_t)kListCap || total > (uint32_t)kListCap - base) return;
  uint64_t* list = ws.lists + r * kListCap + base + before;
  for (uint32_t i = lane; i < off; i += 64) {
    list[i] = ((uint64_t)radix_key(__uint_as_float(staged[0][i])) << 32) | (uint64_t)staged[1][i];
  }
}

// LDS of topk_digit_finish: its one-pass counting sort, or (fallback) the
// refine-and-sort state of select_row.
struct FinishSort {
  uint64_t sorted[kSortCap];
  uint64_t out[kMaxK];
  uint32_t start[kSortBins];   // keys in higher buckets
  uint32_t cursor[kSortBins];  // bucket counts, then scatter cursors
  uint32_t wave_sums[kThreads / 64];
  uint32_t crowded;
  uint32_t bound;     // the bucket holding sorted position count - 1
  uint32_t live_end;  // the end of that bucket: keys past it are not sorted
};
union FinishShared {
  Shared sh;
  FinishSort fs;
};

// One counting sort of the n candidate keys (unique composite keys whose
// radix keys lie in [lo, hi]) held kSortPerThread per thread (slot j of a
// thread holds a key when bit j of `valid` is set): kSortBins linear
// buckets of the radix keys,
// ranks inside a bucket by comparison, the first `count` through LDS to
// emit(i, key). Buckets that start at or past `count` hold no output key and
// are neither ranked nor limited in size. fs.cursor and fs.crowded must be
// zero on entry. Returns false, with nothing emitted, when a bucket that
// starts below `count` holds more than kSortBucketMax keys.
template <typename Emit>
__device__ __forceinline__ bool counting_sort_mask(FinishSort& fs, const uint64_t (&key)[kSortPerThread],
                                                   uint32_t valid, uint32_t n, uint32_t lo,
                                                   uint32_t hi, int count, Emit&& emit) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Linear buckets over the radix keys [lo, hi], descending order =
  // descending bucket, then descending key.
  const uint32_t span = hi - lo + 1u;  // 0 stands for 2^32
  const int bits = 32 - __builtin_clz((span - 1) | 1u);
  const int shift = bits > 12 ? bits - 12 : 0;
  // (Clamped: keys outside the range only come with counts that disagree
  // with the scores, and must not index outside the buckets.)
  auto bucket_of = [lo, shift](uint64_t k) {
    return min(((uint32_t)(k >> 32) - lo) >> shift, (uint32_t)kSortBins - 1);
  };
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j)
    if ((valid >> j) & 1u) atomicAdd(&fs.cursor[bucket_of(key[j])], 1u);
  __syncthreads();
  // Thread t owns buckets 4t .. 4t + 3; start = keys in higher buckets.
  uint32_t c4[4], own = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c4[j] = fs.cursor[4 * tid + j];
    own += c4[j];
  }
  // Keys in buckets of this and higher threads of the wave.
  const uint32_t incl = logits_core::wave_suffix_sum(own);
  if (lane == 0) fs.wave_sums[wave] = incl;
  __syncthreads();
  // Keys of the higher waves: one read of the wave totals per wave (lanes
  // 0-15), their suffix sum, then lane wave + 1's.
  const uint32_t totals = logits_core::wave_suffix_sum(lane < kThreads / 64 ? fs.wave_sums[lane] : 0u);
  uint32_t higher = incl - own + __builtin_amdgcn_readlane(totals, wave + 1);
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    fs.start[4 * tid + j] = higher;
    fs.cursor[4 * tid + j] = higher;
    if (c4[j] > kSortBucketMax && higher < (uint32_t)count) fs.crowded = 1;
    if (higher < (uint32_t)count && higher + c4[j] >= (uint32_t)count) {
      fs.bound = 4 * tid + j;
      fs.live_end = higher + c4[j];
    }
    higher += c4[j];
  }
  __syncthreads();
  if (!fs.crowded) {
    // Buckets below the one holding position count - 1 start at or past
    // `count` and hold no output key: their keys are neither placed nor
    // ranked.
    const uint32_t bound = fs.bound, live_end = fs.live_end;
#pragma unroll
    for (int j = 0; j < kSortPerThread; ++j) {
      const uint32_t b = bucket_of(key[j]);
      if (((valid >> j) & 1u) && b >= bound) fs.sorted[atomicAdd(&fs.cursor[b], 1u)] = key[j];
    }
    __syncthreads();
    // Rank inside the bucket; bucket b spans [start[b], start[b - 1]).
    for (uint32_t i = tid; i < live_end; i += kThreads) {
      const uint64_t k = fs.sorted[i];
      const uint32_t b = bucket_of(k);
      const uint32_t b0 = fs.start[b], b1 = b ? fs.start[b - 1] : n;
      uint32_t rank = b0, j = b0;
      for (; j + 4 <= b1; j += 4) {
        const uint64_t x0 = fs.sorted[j], x1 = fs.sorted[j + 1];
        const uint64_t x2 = fs.sorted[j + 2], x3 = fs.sorted[j + 3];
        rank += (x0 > k ? 1u : 0u) + (x1 > k ? 1u : 0u) + (x2 > k ? 1u : 0u) + (x3 > k ? 1u : 0u);
      }
      for (; j < b1; ++j) rank += fs.sorted[j] > k ? 1u : 0u;
      if (rank < (uint32_t)count) fs.out[rank] = k;
    }
    __syncthreads();
    for (int i = tid; i < count; i += kThreads) emit(i, fs.out[i]);
    return true;
  }
  return false;
}

// The same with the keys at positions t + j kThreads < n.
__device__ __forceinline__ uint32_t prefix_slots(uint32_t n) {
  uint32_t valid = 0;
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j)
    valid |= (int)threadIdx.x + j * kThreads < (int)n ? 1u << j : 0u;
  return valid;
}
template <typename Emit>
__device__ __forceinline__ bool counting_sort_range(FinishSort& fs, const uint64_t (&key)[kSortPerThread],
                                                    uint32_t n, uint32_t lo, uint32_t hi, int count,
                                                    Emit&& emit) {
  return counting_sort_mask(fs, key, prefix_slots(n), n, lo, hi, count, emit);
}

// The same over every key at or above digit d0, top the highest digit.
template <typename Emit>
__device__ __forceinline__ bool counting_sort_keys(FinishSort& fs, const uint64_t (&key)[kSortPerThread],
                                                   uint32_t n, uint32_t d0, uint32_t top, int count,
                                                   Emit&& emit) {
  return counting_sort_range(fs, key, n, d0 << 21, ((top + 1) << 21) - 1u, count, emit);
}

// One work-group per row, after topk_digit_select. Zeroes the row's counts
// and fill, then sorts the listed candidates (every key at or above the
// threshold digit, held kSortPerThread per thread) by one counting sort over
// kSortBins linear buckets of their radix keys between the threshold digit
// and the top digit, and writes the first `count` of them. With a bucket of
// more than kSortBucketMax keys, or an incomplete list, it splits the
// threshold digit's keys first (in LDS, or over the row when they exceed
// kRefineCap or were not listed) and sorts the `count` keys as select_row
// does. A row whose counts do not sum to its columns runs select_row over
// its scores.
__global__ __launch_bounds__(kThreads, 1) void topk_digit_finish(const float* __restrict__ scores,
                                                                int64_t cols, int64_t ld,
                                                                int total_count,
                                                                float* __restrict__ values,
                                                                int32_t* __restrict__ ids,
                                                                int64_t out_ld, DigitWorkspace ws,
                                                                bool listed) {
  __shared__ FinishShared lds;
  __shared__ uint32_t info[6];  // valid, digit, above, bucket, top, fill
  FinishSort& fs = lds.fs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t r = blockIdx.x;
  const int count = total_count < cols ? total_count : (int)cols;
  uint32_t* row_counts = ws.counts + r * kBins;
  const uint64_t* list = ws.lists + r * kListCap;
  // One round of loads: the threshold record, the fill and the first
  // kSortEager key slots of every thread (the list is that long whatever
  // its fill, so these loads stay inside it).
  uint64_t key[kSortPerThread];
#pragma unroll
  for (int j = 0; j < kSortEager; ++j) key[j] = list[tid + j * kThreads];
  if (!listed) {
    // No selection launch ran: the threshold comes from the counts here.
    if (tid < 64) {
      const Threshold t = row_threshold(row_counts, (uint32_t)count);
      if (lane == 0) {
        info[0] = t.total == (uint32_t)cols;
        info[1] = t.digit;
        info[2] = t.above;
        info[3] = t.bucket;
        info[4] = t.top;
        info[5] = 0;
      }
    }
  } else if (tid < 5) {
    info[tid] = ws.threshold[r * 8 + tid];
  } else if (tid == 5) {
    info[5] = ws.fill[r];
  }
  for (int i = tid; i < kSortBins; i += kThreads) fs.cursor[i] = 0;
  if (tid == 0) fs.crowded = 0;
  __syncthreads();
  for (int i = tid; i < kBins; i += kThreads) row_counts[i] = 0;
  if (tid == 0) ws.fill[r] = 0;
  if (count >= cols || !info[0]) {
    select_row<kResidentVecSmall>(lds.sh, scores, cols, ld, total_count, values, ids, out_ld,
                                  nullptr, r, 0, 1);
    return;
  }
  const uint32_t d0 = info[1], above = info[2], bucket = info[3], top = info[4];
  const uint32_t n = above + bucket;
  const bool complete = listed && info[5] == n;
  float* vout = values + r * out_ld;
  int32_t* iout = ids + r * out_ld;
  auto emit = [&](int i, uint64_t k) {
    const uint32_t b = key_bits((uint32_t)(k >> 32));
    vout[i] = __uint_as_float(b);
    const bool finite = (b & 0x7F800000u) != 0x7F800000u;
    iout[i] = finite ? (int32_t)(~(uint32_t)k) : -1;
  };
  if (complete) {
    if (n > (uint32_t)(kSortEager * kThreads)) {
#pragma unroll
      for (int j = kSortEager; j < kSortPerThread; ++j) key[j] = list[tid + j * kThreads];
    }
    if (counting_sort_keys(fs, key, n, d0, top, count, emit)) return;
    __syncthreads();  // before the fallback reuses the LDS
  }
  // Fallback: split the threshold digit's keys to exactly `count` keys, then sort.
  Shared& sh = lds.sh;
  const uint64_t prefix = (uint64_t)d0 << kShift[0];
  const uint32_t remaining = (uint32_t)count - above;
  if (tid == 0) {
    sh.n_sel = 0;
    sh.n_buf = 0;
  }
  __syncthreads();
  if (complete && bucket <= (uint32_t)kRefineCap) {
#pragma unroll
    for (int j = 0; j < kSortPerThread; ++j) {
      const bool live = tid + j * kThreads < (int)n;
      const bool is_above = live && (key[j] >> kShift[0]) > d0;
      const bool in_bucket = live && !is_above;
      const uint32_t slot_above = wave_slot(&sh.n_sel, is_above);
      const uint32_t slot_bucket = wave_slot(&sh.n_buf, in_bucket);
      if (is_above && slot_above < (uint32_t)kMaxK) sh.sel[slot_above] = key[j];
      if (in_bucket && slot_bucket < (uint32_t)kRefineCap) sh.buf[slot_bucket] = key[j];
    }
    __syncthreads();
    refine_buffer(sh, prefix, kShift[0], remaining, bucket == remaining, bucket);
  } else {
    const float* row = scores + r * ld;
    refine_from_row(sh, row, cols, (reinterpret_cast<uintptr_t>(row) & 15) == 0, prefix,
                    kShift[0], remaining, bucket == remaining);
  }
  __syncthreads();
  sort_selected(sh, count);
  for (int i = tid; i < count; i += kThreads) emit(i, sh.sel[i]);
}

// ---- exact top-k from the candidates of the fused indexer step.
//
// The logits kernel's candidate mode (logits.hip) leaves, per row r with a
// floor F > 0: for each key split, a list of the composite keys of the
// split's scores at or above F, and from the split's spill column on (when
// its list would overflow) the split's scores stored in full in the score
// row. A row with F = 0 was stored in full. The candidates - listed keys and
// spilled scores at or above F - hold every score of the row at or above F,
// so when there are at least `count` of them they hold the row's top
// `count` (and the top-k of the candidates is the row's). When there are
// more than the sort holds, the floor is raised to the level-0 digit of the
// count-th largest candidate and the candidates are listed again. Otherwise
// (F was above the row's count-th largest score, or the raised floor still
// leaves too many), the row's scores are recomputed here with the logits
// kernel's arithmetic (logits_core.h) and selected from in full.
struct CandidateLists {
  const uint32_t* floors;   // [rows][2] the row's floor (row_floor), 0 when stored in full
  const uint32_t* records;  // [rows][splits][2]: keys listed, first spilled column
  const uint64_t* lists;    // [rows][splits][cap] composite keys
  int64_t splits, per, cap;
};
struct LogitsInputs {
  const uint8_t* q;
  const uint8_t* k;
  const float* w;
  const float* kscale;
  const int32_t* starts;
  const int32_t* ends;
  int64_t query_start;
  const float* q_fold;
};
constexpr int kMaxCandidateSplits = 512;

__global__ __launch_bounds__(kThreads, 1) void topk_candidates(float* __restrict__ scores,
                                                              int64_t cols, int64_t ld,
                                                              int total_count,
                                                              float* __restrict__ values,
                                                              int32_t* __restrict__ ids,
                                                              int64_t out_ld, CandidateLists cl,
                                                              LogitsInputs li) {
  __shared__ FinishShared lds;
  __shared__ uint32_t info[8];  // fill, largest radix key, -, digit, above, bucket
  __shared__ uint4 wave_parts[kThreads / 64];  // per wave: listed keys, largest radix key, misfit
  FinishSort& fs = lds.fs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t r = blockIdx.x;
  const int count = total_count < cols ? total_count : (int)cols;

  // The split records and the first list entries are loaded first, before
  // anything waits on memory: thread t serves key split t / T (T = kThreads /
  // splits threads per split) and loads entries u, u + T, ... (u = t % T) of
  // its first kSpecSlots slots whatever the record says (entries below the
  // list's capacity, so in bounds; slots past the list's length are wasted
  // reads, so not all kSortPerThread are loaded blind); the later slots
  // follow once the record says they are listed. On the fast path - no split
  // spilled and every list fits its threads' kSortPerThread slots - the
  // listed ones go straight into the sort's registers.
  constexpr int kWaves = kThreads / 64;
  const int splits = (int)cl.splits;
  const int per_split = kThreads / splits;  // >= 2 (splits <= 512)
  const int sp = tid / per_split, u = tid % per_split;
  const bool sp_live = sp < splits && (int64_t)sp * cl.per < cols;
  const int64_t sp_at = r * cl.splits + (sp_live ? sp : 0);
  uint64_t key[kSortPerThread];
  uint32_t rec0, rec1;
  {
    const uint32_t* rec = cl.records + sp_at * 2;
    rec0 = rec[0];
    rec1 = rec[1];
    const uint64_t* src = cl.lists + sp_at * cl.cap;
#pragma unroll
    for (int j = 0; j < kSpecSlots; ++j) {
      const int64_t e = u + (int64_t)per_split * j;
      key[j] = src[e < cl.cap ? e : cl.cap - 1];  // unused past the capacity
    }
  }
  const uint32_t floor = logits_core::row_floor(cl.floors, r);
  uint32_t sort_lo = floor;  // the smallest radix key the sort can meet
  // The loads stay above the floor test: without these uses the compiler
  // sinks them into the branch that reads them, behind the floor's wait.
  asm volatile("" : "+v"(rec0), "+v"(rec1));
#pragma unroll
  for (int j = 0; j < kSpecSlots; ++j) asm volatile("" : "+v"(key[j]));
  if (floor == 0) {
    select_row<kResidentVecSmall>(lds.sh, scores, cols, ld, total_count, values, ids, out_ld,
                                  nullptr, r, 0, 1);
    return;
  }
  const int64_t vis_lo = li.starts ? (int64_t)li.starts[r] : 0;
  int64_t vis_hi = li.ends ? (int64_t)li.ends[r] : li.query_start + r + 1;
  if (vis_hi > cols) vis_hi = cols;
  float* row = scores + r * ld;
  float* vout = values + r * out_ld;
  int32_t* iout = ids + r * out_ld;
  auto emit = [&](int i, uint64_t k) {
    const uint32_t b = key_bits((uint32_t)(k >> 32));
    vout[i] = __uint_as_float(b);
    const bool finite = (b & 0x7F800000u) != 0x7F800000u;
    iout[i] = finite ? (int32_t)(~(uint32_t)k) : -1;
  };
  for (int i = tid; i < kSortBins; i += kThreads) fs.cursor[i] = 0;
  if (tid == 0) fs.crowded = 0;

  const uint32_t n_sp = sp_live ? rec0 : 0u;
  const int32_t spill_sp = sp_live ? (int32_t)rec1 : 0x7FFFFFFF;
  const bool fits = spill_sp == 0x7FFFFFFF && n_sp <= (uint32_t)(per_split * kSortPerThread);
  {
    const uint64_t* src = cl.lists + sp_at * cl.cap;
#pragma unroll
    for (int j = kSpecSlots; j < kSortPerThread; ++j) {
      const uint32_t e = (uint32_t)(u + per_split * j);
      key[j] = fits && e < n_sp ? src[e] : 0ull;
    }
  }
  uint32_t valid = 0, top_key = 0;
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j) {
    const uint32_t e = (uint32_t)(u + per_split * j);
    const bool live = fits && e < n_sp;
    key[j] = live ? key[j] : 0ull;
    valid |= live ? 1u << j : 0u;
    top_key = max(top_key, (uint32_t)(key[j] >> 32));
  }
  {
    uint32_t total = 0;
    (void)wave_prefix_any(u == 0 ? n_sp : 0u, &total);
    const bool misfit = __builtin_amdgcn_ballot_w64(!fits) != 0;
    top_key = max(top_key, lane_xor<1>(top_key));
    top_key = max(top_key, lane_xor<2>(top_key));
    top_key = max(top_key, lane_xor<4>(top_key));
    top_key = max(top_key, lane_xor<8>(top_key));
    top_key = max(top_key, lane_xor<16>(top_key));
    top_key = max(top_key, lane_xor<32>(top_key));
    if (lane == 0) wave_parts[wave] = uint4{total, top_key, misfit ? 1u : 0u, 0u};
  }
  __syncthreads();  // the wave parts and the LDS state above are set
  // The totals: lanes 0-15 of each wave read one wave's part each.
  uint32_t n_cand, top_all;
  bool misfit_any;
  {
    const uint4 part = lane < kWaves ? wave_parts[lane] : uint4{0u, 0u, 0u, 0u};
    uint32_t tot = part.x, top = part.y;
    // row_shl:k (0x100 + k): lane l reads lane l + k of its 16-lane row, 0 past it.
    tot += __builtin_amdgcn_update_dpp(0u, tot, 0x101, 0xF, 0xF, false);
    top = max(top, (uint32_t)__builtin_amdgcn_update_dpp(0u, top, 0x101, 0xF, 0xF, false));
    tot += __builtin_amdgcn_update_dpp(0u, tot, 0x102, 0xF, 0xF, false);
    top = max(top, (uint32_t)__builtin_amdgcn_update_dpp(0u, top, 0x102, 0xF, 0xF, false));
    tot += __builtin_amdgcn_update_dpp(0u, tot, 0x104, 0xF, 0xF, false);
    top = max(top, (uint32_t)__builtin_amdgcn_update_dpp(0u, top, 0x104, 0xF, 0xF, false));
    tot += __builtin_amdgcn_update_dpp(0u, tot, 0x108, 0xF, 0xF, false);
    top = max(top, (uint32_t)__builtin_amdgcn_update_dpp(0u, top, 0x108, 0xF, 0xF, false));
    n_cand = __builtin_amdgcn_readfirstlane(tot);
    top_all = __builtin_amdgcn_readfirstlane(top);
    misfit_any = __builtin_amdgcn_ballot_w64(part.z != 0u) != 0;
  }
  if (misfit_any) {
    // Candidates into the LDS buffer in no order (the sort does not need
    // one): wave w takes the key splits w, w + 16, ... - lane j holds split
    // w + 16 j's record - and one LDS atomic places all their listed keys;
    // the lists are copied in chunks of 64 keys, eight chunks of loads in
    // flight at a time. Spilled scores at or above the floor follow.
    if (tid == 0) {
      info[0] = 0;        // fill
      info[1] = top_all;  // largest radix key
    }
    __syncthreads();
    const int my_split = wave + kWaves * lane;
    uint32_t n_l = 0;
    int32_t spill_l = 0x7FFFFFFF;
    if (my_split < splits && (int64_t)my_split * cl.per < cols) {
      const uint32_t* rec = cl.records + (r * cl.splits + my_split) * 2;
      n_l = rec[0];
      spill_l = (int32_t)rec[1];
    }
    uint32_t n_wave = 0;
    const uint32_t n_pre = wave_prefix_any(n_l, &n_wave);
    uint32_t chunks_wave = 0;
    const uint32_t chunks_l = (n_l + 63) / 64;
    const uint32_t chunk_pre = wave_prefix_any(chunks_l, &chunks_wave);
    uint32_t wave_base = 0;
    if (lane == 0 && n_wave) wave_base = atomicAdd(&info[0], n_wave);
    wave_base = __builtin_amdgcn_readfirstlane(wave_base);
    const int wave_splits = (splits - wave + kWaves - 1) / kWaves;  // lanes holding a split
    uint32_t top = 0;
    constexpr int kChunks = 8;
    for (uint32_t c0 = 0; c0 < chunks_wave; c0 += kChunks) {
      uint64_t v[kChunks];
      uint32_t dst[kChunks];
      bool ok[kChunks];
#pragma unroll
      for (int q = 0; q < kChunks; ++q) {
        const uint32_t c = c0 + q;
        // The lane whose split holds chunk c (wave-uniform search).
        int j = 0;
        for (int t = 1; t < wave_splits && t < 64; ++t)
          if (__builtin_amdgcn_readlane(chunk_pre, t) <= c) j = t;
        const uint32_t n_j = __builtin_amdgcn_readlane(n_l, j);
        const uint32_t i = 64 * (c - __builtin_amdgcn_readlane(chunk_pre, j)) + lane;
        ok[q] = c < chunks_wave && i < n_j;
        const uint64_t* src = cl.lists + (r * cl.splits + wave + kWaves * j) * cl.cap;
        v[q] = ok[q] ? src[i] : 0ull;
        dst[q] = wave_base + __builtin_amdgcn_readlane(n_pre, j) + i;
      }
#pragma unroll
      for (int q = 0; q < kChunks; ++q)
        if (ok[q] && dst[q] < (uint32_t)kSortCap) fs.sorted[dst[q]] = v[q];
    }
    for (int j = 0; j < wave_splits && j < 64; ++j) {
      const int32_t spill = __builtin_amdgcn_readlane(spill_l, j);
      if (spill == 0x7FFFFFFF) continue;
      const int64_t kb = (int64_t)(wave + kWaves * j) * cl.per;
      int64_t lo = spill, hi = kb + cl.per;
      if (lo < vis_lo) lo = vis_lo;
      if (hi > vis_hi) hi = vis_hi;
      for (int64_t c0 = lo; c0 < hi; c0 += 64) {
        const int64_t c = c0 + lane;
        const float v = c < hi ? row[c] : 0.0f;
        const uint32_t k = radix_key(v);
        const bool hit = c < hi && k >= floor;
        const uint32_t slot = wave_slot(&info[0], hit);
        if (hit && slot < (uint32_t)kSortCap) fs.sorted[slot] = composite(v, c);
        if (hit) top = max(top, k);
      }
    }
    top = max(top, lane_xor<1>(top));
    top = max(top, lane_xor<2>(top));
    top = max(top, lane_xor<4>(top));
    top = max(top, lane_xor<8>(top));
    top = max(top, lane_xor<16>(top));
    top = max(top, lane_xor<32>(top));
    if (lane == 0) atomicMax(&info[1], top);
    __syncthreads();
    n_cand = info[0];
    top_all = info[1];
    if (n_cand > (uint32_t)kSortCap && n_cand >= (uint32_t)count) {
      // More candidates than the sort holds (the floor was low): raise the
      // floor to the level-0 digit of the row's count-th largest candidate,
      // from a histogram of all of them, and list again those at or above
      // it. Each pass streams the lists and the spilled scores as above.
      auto stream = [&](auto&& sink) __attribute__((always_inline)) {
        for (uint32_t c0 = 0; c0 < chunks_wave; c0 += kChunks) {
          uint64_t v[kChunks];
          bool ok[kChunks];
#pragma unroll
          for (int q = 0; q < kChunks; ++q) {
            const uint32_t c = c0 + q;
            int j = 0;
            for (int t = 1; t < wave_splits && t < 64; ++t)
              if (__builtin_amdgcn_readlane(chunk_pre, t) <= c) j = t;
            const uint32_t n_j = __builtin_amdgcn_readlane(n_l, j);
            const uint32_t i = 64 * (c - __builtin_amdgcn_readlane(chunk_pre, j)) + lane;
            ok[q] = c < chunks_wave && i < n_j;
            const uint64_t* src = cl.lists + (r * cl.splits + wave + kWaves * j) * cl.cap;
            v[q] = ok[q] ? src[i] : 0ull;
          }
#pragma unroll
          for (int q = 0; q < kChunks; ++q) sink(ok[q], v[q]);
        }
        for (int j = 0; j < wave_splits && j < 64; ++j) {
          const int32_t spill = __builtin_amdgcn_readlane(spill_l, j);
          if (spill == 0x7FFFFFFF) continue;
          const int64_t kb = (int64_t)(wave + kWaves * j) * cl.per;
          int64_t lo = spill, hi = kb + cl.per;
          if (lo < vis_lo) lo = vis_lo;
          if (hi > vis_hi) hi = vis_hi;
          for (int64_t c0 = lo; c0 < hi; c0 += 64) {
            const int64_t c = c0 + lane;
            const float v = c < hi ? row[c] : 0.0f;
            sink(c < hi && radix_key(v) >= floor, composite(v, c));
          }
        }
      };
      for (int i = tid; i < kBins; i += kThreads) fs.start[i] = 0;
      __syncthreads();
      stream([&](bool ok, uint64_t k) {
        if (ok) atomicAdd(&fs.start[k >> 53], 1u);
      });
      __syncthreads();
      if (wave == 0) {
        const Threshold t = row_threshold(fs.start, (uint32_t)count);
        if (lane == 0) {
          info[3] = t.digit;
          info[4] = t.above + t.bucket;
        }
      }
      if (tid == 0) info[0] = 0;
      __syncthreads();
      if (info[4] <= (uint32_t)kSortCap) {
        const uint32_t raised = max(floor, info[3] << 21);
        stream([&](bool ok, uint64_t k) {
          const bool keep = ok && (uint32_t)(k >> 32) >= raised;
          const uint32_t slot = wave_slot(&info[0], keep);
          if (keep && slot < (uint32_t)kSortCap) fs.sorted[slot] = k;
        });
        __syncthreads();
        n_cand = info[0];  // == info[4]
        sort_lo = raised;
      }
    }
    valid = n_cand <= (uint32_t)kSortCap ? prefix_slots(n_cand) : 0u;
#pragma unroll
    for (int j = 0; j < kSortPerThread; ++j)
      key[j] = (valid >> j) & 1u ? fs.sorted[tid + j * kThreads] : 0ull;
    __syncthreads();  // the sort scatters into the buffer
  }
  // Fewer than `count` candidates: the floor was above the count-th
  // largest score, and scores below it are missing.
  if (n_cand <= (uint32_t)kSortCap && n_cand >= (uint32_t)count) {
    if (counting_sort_mask(fs, key, valid, n_cand, sort_lo, top_all, count, emit)) return;
    // A crowded bucket: the threshold digit from the candidates' digit
    // histogram, then its keys split to exactly count - above (select_row's
    // refinement).
    __syncthreads();
    for (int i = tid; i < kBins; i += kThreads) fs.start[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortPerThread; ++j)
      if ((valid >> j) & 1u) atomicAdd(&fs.start[key[j] >> 53], 1u);
    __syncthreads();
    if (wave == 0) {
      const Threshold t = row_threshold(fs.start, (uint32_t)count);
      if (lane == 0) {
        info[3] = t.digit;
        info[4] = t.above;
        info[5] = t.bucket;
      }
    }
    __syncthreads();
    const uint32_t d0 = info[3], above = info[4], bucket = info[5];
    if (bucket <= (uint32_t)kRefineCap) {
      Shared& sh = lds.sh;
      if (tid == 0) {
        sh.n_sel = 0;
        sh.n_buf = 0;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kSortPerThread; ++j) {
        const bool live = (valid >> j) & 1u;
        const uint32_t digit = (uint32_t)(key[j] >> kShift[0]);
        const bool is_above = live && digit > d0;
        const bool in_bucket = live && digit == d0;
        const uint32_t slot_above = wave_slot(&sh.n_sel, is_above);
        const uint32_t slot_bucket = wave_slot(&sh.n_buf, in_bucket);
        if (is_above && slot_above < (uint32_t)kMaxK) sh.sel[slot_above] = key[j];
        if (in_bucket && slot_bucket < (uint32_t)kRefineCap) sh.buf[slot_bucket] = key[j];
      }
      __syncthreads();
      const uint32_t remaining = (uint32_t)count - above;
      refine_buffer(sh, (uint64_t)d0 << kShift[0], kShift[0], remaining, bucket == remaining, bucket);
      __syncthreads();
      sort_selected(sh, count);
      for (int i = tid; i < count; i += kThreads) emit(i, sh.sel[i]);
      return;
    }
    // A threshold digit of more than kRefineCap keys: from the full row.
  }
  // The row's exact scores (every column), then the selection over them.
  __syncthreads();
  uint8_t(*digits)[logits_core::kDigits][logits_core::kDim] =
      reinterpret_cast<uint8_t(*)[logits_core::kDigits][logits_core::kDim]>(
          reinterpret_cast<uint8_t*>(&lds) +
          wave * logits_core::kQueriesPerWave * logits_core::kDigits * logits_core::kDim);
  logits_core::row_scores(li.q, li.k, li.w, li.kscale, li.q_fold, r, (int32_t)vis_lo,
                          (int32_t)vis_hi, cols, row, digits, wave, kThreads / 64);
  __syncthreads();
  select_row<kResidentVecSmall>(lds.sh, scores, cols, ld, total_count, values, ids, out_ld,
                                nullptr, r, 0, 1);
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
  auto kernel = columns <= resident_cols(kResidentVecSmall) ? topk_rows<kResidentVecSmall>
                                                             : topk_rows<kResidentVecLarge>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)rows, 1), dim3(kThreads), 0, stream, scores, columns,
                     ld, (int)count, values, indices, out_ld, nullptr);
  DSA_CHECK_LAUNCH("exact top-k");
  return kOk;
}


extern "C" int dsa_indexer_topk_workspace_bytes(int64_t rows, int64_t columns, int64_t* bytes) {
  using namespace dsa;
  DSA_CHECK_ARG(rows >= 0 && rows < 0x7FFFFFFF && columns >= 1 && columns < 0x7FFFFFFF &&
                    bytes != nullptr,
                "invalid indexer top-k workspace query");
  *bytes = digit_workspace_bytes(rows, columns);
  return kOk;
}

extern "C" int dsa_topk_radix_digits(const float* scores, int64_t rows, int64_t columns,
                                     int64_t ld, int64_t k, float* values, int32_t* indices,
                                     int64_t out_ld, void* workspace, int64_t workspace_bytes,
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
  DSA_CHECK_ARG(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 8 == 0 &&
                    workspace_bytes >= digit_workspace_bytes(rows, columns),
                "indexer top-k workspace too small or misaligned");
  const DigitWorkspace ws = digit_workspace(workspace, rows, columns);
  // Rows of more than 64 parts are split over their scores by the finish
  // kernel alone (no selection launch).
  const bool listed = ws.parts <= 64;
  if (count < columns && listed) {
    const int64_t part_cols = ((columns + ws.parts - 1) / ws.parts + 3) & ~(int64_t)3;
    hipLaunchKernelGGL(topk_digit_select, dim3((unsigned)rows, (unsigned)ws.parts), dim3(kThreads),
                       0, stream, scores, columns, ld, (int)count, part_cols, ws);
    DSA_CHECK_LAUNCH("exact top-k");
  }
  hipLaunchKernelGGL(topk_digit_finish, dim3((unsigned)rows), dim3(kThreads), 0, stream, scores,
                     columns, ld, (int)count, values, indices, out_ld, ws, listed);
  DSA_CHECK_LAUNCH("exact top-k");
  return kOk;
}

namespace dsa {

int topk_from_candidates(const uint8_t* q, const uint8_t* k, const float* weights,
                         const float* kscale, const int32_t* starts, const int32_t* ends,
                         int64_t query_start, const float* q_fold, float* scores, int64_t rows,
                         int64_t columns, int64_t ld, int64_t topk, float* values,
                         int32_t* indices, int64_t out_ld, const uint32_t* floors,
                         const uint32_t* records, const uint64_t* lists, int64_t splits,
                         int64_t per, int64_t cap, hipStream_t stream) {
  DSA_CHECK_ARG(splits >= 1 && splits <= kMaxCandidateSplits, "too many key splits");
  DSA_CHECK_ARG(columns < (int64_t)0x7FFFFFFF && rows < 0x7FFFFFFF, "too many rows or columns");
  const int64_t count = topk < columns ? topk : columns;
  hipLaunchKernelGGL(topk_candidates, dim3((unsigned)rows), dim3(kThreads), 0, stream, scores,
                     columns, ld, (int)count, values, indices, out_ld,
                     CandidateLists{floors, records, lists, splits, per, cap},
                     LogitsInputs{q, k, weights, kscale, starts, ends, query_start, q_fold});
  DSA_CHECK_LAUNCH("indexer top-k from candidates");
  return kOk;
}

}  // namespace dsa

namespace dsa {
namespace {
int64_t topk_workspace_bytes(int64_t rows) { return rows * 2 * kMaxK * 8; }
}  // namespace
}  // namespace dsa

extern "C" int dsa_topk_workspace_bytes(int64_t rows, int64_t* bytes) {
  using namespace dsa;
  DSA_CHECK_ARG(rows >= 0 && rows < 0x7FFFFFFF && bytes != nullptr, "invalid top-k workspace query");
  *bytes = topk_workspace_bytes(rows);
  return kOk;
}

extern "C" int dsa_topk_radix_split(const float* scores, int64_t rows, int64_t columns, int64_t ld,
                                    int64_t k, float* values, int32_t* indices, int64_t out_ld,
                                    void* workspace, int64_t workspace_bytes, hipStream_t stream) {
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
  // Rows too short to be worth two work-groups take the one-part kernel.
  if (columns < 4 * kMaxK) return dsa_topk_radix(scores, rows, columns, ld, k, values, indices, out_ld, stream);
  DSA_CHECK_ARG(workspace != nullptr && workspace_bytes >= topk_workspace_bytes(rows),
                "top-k workspace too small");
  DSA_CHECK_ARG(reinterpret_cast<uintptr_t>(workspace) % 8 == 0, "workspace must be 8-byte aligned");
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const int64_t part_cols = (((columns + 1) >> 1) + 3) & ~(int64_t)3;
  auto kernel = part_cols <= resident_cols(kResidentVecSmall) ? topk_rows<kResidentVecSmall>
                                                               : topk_rows<kResidentVecLarge>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)rows, 2), dim3(kThreads), 0, stream, scores, columns,
                     ld, (int)count, values, indices, out_ld, keys);
  DSA_CHECK_LAUNCH("exact top-k");
  hipLaunchKernelGGL(topk_merge, dim3((unsigned)rows), dim3(kThreads), 0, stream, keys, columns,
                     (int)count, values, indices, out_ld);
  DSA_CHECK_LAUNCH("exact top-k");
  return kOk;
}

// ---- the same two-part top-k with its half-row lists in a library-owned
// device array instead of a caller workspace, for callers that cannot
// allocate. `scratch` is a host-side stand-in in host code: its device
// address on each GPU comes from hipGetSymbolAddress, resolved once per
// device with that device current, and only that address is passed to the
// kernels. Every call on one GPU shares that GPU's array.
namespace dsa {
namespace {
constexpr int64_t kStaticTopkRows = 512;
__device__ __align__(256) uint64_t scratch[kStaticTopkRows * 2 * kMaxK];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
uint64_t* scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(uint64_t** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) {
    set_error("hipGetDevice failed: %s", hipGetErrorString(err));
    return kLaunchFailed;
  }
  DSA_CHECK_ARG(device >= 0 && device < kMaxDevices, "device ordinal %d out of range", device);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                hipGetErrorString(err));
      return kLaunchFailed;
    }
    scratch_ptr[device] = static_cast<uint64_t*>(ptr);
  }
  *out = scratch_ptr[device];
  return kOk;
}
}  // namespace
}  // namespace dsa

extern "C" int dsa_topk_radix_split_static(const float* scores, int64_t rows, int64_t columns,
                                           int64_t ld, int64_t k, float* values,
                                           int32_t* indices, int64_t out_ld,
                                           hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(rows >= 0 && rows <= kStaticTopkRows,
                "dsa_topk_radix_split_static handles at most %lld rows per call (got %lld)",
                (long long)kStaticTopkRows, (long long)rows);
  if (rows == 0 || columns < 4 * kMaxK)
    return dsa_topk_radix_split(scores, rows, columns, ld, k, values, indices, out_ld, nullptr, 0,
                                stream);
  uint64_t* keys = nullptr;
  const int status = scratch_for_current_device(&keys);
  if (status != kOk) return status;
  return dsa_topk_radix_split(scores, rows, columns, ld, k, values, indices, out_ld, keys,
                              (int64_t)sizeof(scratch), stream);
}
