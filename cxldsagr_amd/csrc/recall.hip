// A10: exact recall of a top-k selection into a bounded HBM token pool.
//
// Semantics: cache/sparse_token_cache.py:502-569 (ensure) with its victim
// choice _available_slots/_evict (:465-500) and the pool's FIFO events
// (cache/sparse_token_pool.py:648-676):
//   union of selected history ids -> global host ids through the page table
//   -> hits get priority = protect_stamp; misses (ascending logical order)
//   -> victims = first m available slots by (rank, slot), rank = -1 for an
//   empty slot else its priority; the sentinel slot 0 and this selection's
//   hits are never victims -> evict old owners, publish h2d/d2h, stamp the
//   chosen slots -> gather the missing records from pinned host memory
//   -> map every selected id to its physical slot.
//
// Everything runs on the stream with the miss count kept on the device, so
// there is no host read when the history fits the pool (then every union
// fits too). The (rank, slot) order is one rocPRIM radix sort of 64-bit keys
// over the pool's slots (on the rank bits only: the keys arrive in slot
// order and the sort is stable), the role CUB's radix sort plays in the reference
// (operators/deepseek_v32/indexer/csrc/echo_sparse_recall.cuh:191).
#include <cstring>
#include <mutex>
#include <rocprim/device/device_radix_sort.hpp>

#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

constexpr int32_t kMissing = 0x7FFFFFFF;
constexpr int kPage = 64;
constexpr int kClassifyThreads = 1024;
constexpr int kGatherBlocks = 128;

enum Counter { kUnion = 0, kMisses = 1, kEvicted = 2, kCounters = 4 };
enum StatusBits { kUnwritten = 4, kShortPool = 8 };

__global__ void recall_clear(uint32_t* __restrict__ sel_bits, int64_t sel_words,
                             uint32_t* __restrict__ kept_bits, int64_t kept_words,
                             int64_t* __restrict__ counters) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < sel_words) sel_bits[i] = 0;
  if (i < kept_words) kept_bits[i] = 0;
  if (i < kCounters) counters[i] = 0;
}

__global__ void recall_mark(const int32_t* __restrict__ indices, int64_t n, int64_t history_end,
                            int64_t written, uint32_t* __restrict__ sel_bits,
                            int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t id = indices[i];
  if (id >= written) {
    if (status) atomicOr(status, kUnwritten);
    return;
  }
  if (id >= 0 && id < history_end) atomicOr(&sel_bits[id >> 5], 1u << (id & 31));
}

// recall_mark with the bitmap first built in LDS (a selection repeats ids
// across its rows, so the global words would take ~n / words atomics each):
// each work-group ORs its share of the ids into its own copy, then adds each
// nonzero word to the global bitmap once. For bitmaps of at most
// kMarkLdsWords words.
constexpr int kMarkThreads = 1024;
constexpr int kMarkLdsWords = 8192;    // 262,144 history ids, 32 KB of LDS
constexpr int kMarkIdsPerThread = 8;
constexpr int kMarkIdsPerBlock = kMarkThreads * kMarkIdsPerThread;
__global__ __launch_bounds__(kMarkThreads) void recall_mark_lds(
    const int32_t* __restrict__ indices, int64_t n, int64_t history_end, int64_t written,
    uint32_t* __restrict__ sel_bits, int32_t* __restrict__ status) {
  __shared__ uint32_t local[kMarkLdsWords];
  const int64_t words = (history_end + 31) >> 5;
  for (int64_t w = threadIdx.x; w < words; w += kMarkThreads) local[w] = 0u;
  __syncthreads();
  const int64_t begin = (int64_t)blockIdx.x * kMarkIdsPerBlock + threadIdx.x;
  int64_t ids[kMarkIdsPerThread];
#pragma unroll
  for (int k = 0; k < kMarkIdsPerThread; ++k) {  // all loads first, then the LDS ORs
    const int64_t i = begin + (int64_t)k * kMarkThreads;
    ids[k] = i < n ? indices[i] : -1;
  }
  bool unwritten = false;
#pragma unroll
  for (int k = 0; k < kMarkIdsPerThread; ++k) {
    const int64_t id = ids[k];
    if (id >= written) unwritten = true;
    else if (id >= 0 && id < history_end) atomicOr(&local[id >> 5], 1u << (id & 31));
  }
  if (unwritten && status) atomicOr(status, kUnwritten);
  __syncthreads();
  for (int64_t w = threadIdx.x; w < words; w += kMarkThreads) {
    const uint32_t bits = local[w];
    if (bits) atomicOr(&sel_bits[w], bits);
  }
}

__device__ __forceinline__ int64_t to_global(const int32_t* page_table, int64_t t) {
  return (int64_t)page_table[t / kPage] * kPage + t % kPage;
}

// Hits and misses of the selection, one thread per history id: a selected
// id's global host row through the page table, then h2d; a hit's slot is
// protected (priority = protect_stamp, kept bit), a miss sets its bit in
// miss_bits. The loads of all ids are independent, so they overlap. A wave
// covers two 32-id words and writes them from its ballot.
__global__ __launch_bounds__(256) void recall_lookup(
    const uint32_t* __restrict__ sel_bits, int64_t history_end,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ h2d,
    int64_t* __restrict__ priority, uint32_t* __restrict__ kept_bits, int64_t protect_stamp,
    uint32_t* __restrict__ miss_bits) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool in = t < history_end;
  const uint32_t word = in ? sel_bits[t >> 5] : 0u;
  bool miss = false;
  if ((word >> (t & 31)) & 1u) {
    const int32_t d = h2d[to_global(page_table, t)];
    if (d != kMissing) {
      priority[d] = protect_stamp;
      atomicOr(&kept_bits[d >> 5], 1u << (d & 31));
    } else {
      miss = true;
    }
  }
  const uint64_t m = __builtin_amdgcn_ballot_w64(miss);
  const int64_t words = (history_end + 31) >> 5;
  const int64_t w = (t >> 5);  // lane 0: the wave's first word, lane 32: its second
  if ((lane & 31) == 0 && w < words) miss_bits[w] = (uint32_t)(m >> lane);
}

// One work-group scans the miss bitmap in order: thread t of a round owns
// one 32-id word, and a block scan gives each word the position of its first
// miss in the list (ascending logical order). Also counts the union.
__global__ __launch_bounds__(kClassifyThreads) void recall_classify(
    const uint32_t* __restrict__ sel_bits, const uint32_t* __restrict__ miss_bits,
    int64_t history_end, int32_t* __restrict__ word_offset, int64_t* __restrict__ counters,
    int64_t* __restrict__ stats) {
  __shared__ uint32_t wave_sums[kClassifyThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t words = (history_end + 31) >> 5;
  int64_t running = 0, union_total = 0;
  for (int64_t base = 0; base < words; base += kClassifyThreads) {
    const int64_t w = base + tid;
    const uint32_t bits = w < words ? sel_bits[w] : 0u;
    const uint32_t miss_mask = w < words ? miss_bits[w] : 0u;
    const uint32_t mine = __builtin_popcount(miss_mask);
    uint32_t incl = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wave_sums[wave] = incl;
    uint32_t union_here = __builtin_popcount(bits);
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int i = 0; i < kClassifyThreads / 64; ++i) {
      const uint32_t s = wave_sums[i];
      if (i < wave) before += s;
      total += s;
    }
    if (w < words) word_offset[w] = (int32_t)(running + before + incl - mine);
    running += total;
    // union count: reduce popcounts through the same scratch after a barrier
    __syncthreads();
    uint32_t u = union_here;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) u += __shfl_xor(u, d);
    if (lane == 0) wave_sums[wave] = u;
    __syncthreads();
    for (int i = 0; i < kClassifyThreads / 64; ++i) union_total += wave_sums[i];
    __syncthreads();
  }
  if (tid == 0) {
    counters[kUnion] = union_total;
    counters[kMisses] = running;
    atomicAdd(reinterpret_cast<unsigned long long*>(&stats[0]), (unsigned long long)union_total);
    atomicAdd(reinterpret_cast<unsigned long long*>(&stats[1]), (unsigned long long)running);
  }
}

// The miss list, one thread per history id: a missed id's global host row
// at its word's first position plus the misses before it in the word.
__global__ __launch_bounds__(256) void recall_emit(const uint32_t* __restrict__ miss_bits,
                                                   const int32_t* __restrict__ word_offset,
                                                   int64_t history_end,
                                                   const int32_t* __restrict__ page_table,
                                                   int64_t* __restrict__ misses) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= history_end) return;
  const uint32_t m = miss_bits[t >> 5];
  const uint32_t bit = 1u << (t & 31);
  if (!(m & bit)) return;
  misses[word_offset[t >> 5] + __builtin_popcount(m & (bit - 1u))] = to_global(page_table, t);
}

// Sort keys of the victim order; kept slots (the sentinel, this selection's
// hits and, with keep_floor >= 0, every slot stamped at or after keep_floor)
// sort last and are never chosen.
__global__ void recall_victim_keys(const int64_t* __restrict__ d2h,
                                   const int64_t* __restrict__ priority,
                                   const uint32_t* __restrict__ kept_bits, int64_t slots,
                                   int64_t keep_floor, uint64_t* __restrict__ keys) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (s > slots) return;
  const bool kept = s == 0 || ((kept_bits[s >> 5] >> (s & 31)) & 1u) ||
                    (keep_floor >= 0 && d2h[s] != kMissing && priority[s] >= keep_floor);
  if (kept) {
    keys[s] = ~0ull;
    return;
  }
  const int64_t rank = d2h[s] == kMissing ? -1 : priority[s];
  keys[s] = ((uint64_t)(rank + 1) << 32) | (uint64_t)s;
}

__global__ void recall_assign(const uint64_t* __restrict__ sorted,
                              const int64_t* __restrict__ misses,
                              int64_t* __restrict__ counters, int32_t* __restrict__ h2d,
                              int64_t* __restrict__ d2h, int64_t* __restrict__ priority,
                              int64_t stamp, int64_t* __restrict__ chosen,
                              int64_t* __restrict__ stats, int32_t* __restrict__ status) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t m = counters[kMisses];
  bool evicted = false;
  if (j < m) {
    const uint64_t key = sorted[j];
    if (key == ~0ull) {
      if (status) atomicOr(status, kShortPool);
      chosen[j] = -1;
    } else {
      const int64_t s = (int64_t)(key & 0xFFFFFFFFull);
      const int64_t old = d2h[s];
      if (old != kMissing) {
        h2d[old] = kMissing;
        evicted = true;
      }
      const int64_t g = misses[j];
      d2h[s] = g;
      h2d[g] = (int32_t)s;
      priority[s] = stamp;
      chosen[j] = s;
    }
  }
  // One pair of counter atomics per wave (every lane reaches the ballot).
  const uint64_t ev = __builtin_amdgcn_ballot_w64(evicted);
  if (ev && (threadIdx.x & 63) == 0) {
    const unsigned long long k = (unsigned long long)__builtin_popcountll(ev);
    atomicAdd(reinterpret_cast<unsigned long long*>(&counters[kEvicted]), k);
    atomicAdd(reinterpret_cast<unsigned long long*>(&stats[2]), k);
  }
}

// records[chosen[j]] = host[misses[j]] for j < m; one wave per record.
__global__ __launch_bounds__(256) void recall_gather(const uint8_t* __restrict__ host,
                                                     uint8_t* __restrict__ records,
                                                     const int64_t* __restrict__ misses,
                                                     const int64_t* __restrict__ chosen,
                                                     const int64_t* __restrict__ counters,
                                                     int64_t row_bytes) {
  const int64_t m = counters[kMisses];
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * 4;
  for (int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); j < m; j += stride) {
    const int64_t s = chosen[j];
    if (s < 0) continue;
    const uint4* src = reinterpret_cast<const uint4*>(host + misses[j] * row_bytes);
    uint4* dst = reinterpret_cast<uint4*>(records + s * row_bytes);
    for (int64_t i = lane; i < (row_bytes >> 4); i += 64) dst[i] = src[i];
  }
}

// Selected id -> physical pool row. History ids map through h2d; candidate
// ids (transient_start <= id < written) to rows slots + 1 + candidate_offset
// + id - transient_start, which must lie inside the record rows. Every other id
// (padding, unwritten, past the candidate rows) maps to -1, so that a bad
// selection reads no stale record (recall_mark has flagged it in status).
__global__ void recall_map(const int32_t* __restrict__ indices, int64_t n, int64_t history_end,
                           int64_t written, int64_t transient_start, int64_t slots,
                           int64_t candidate_offset, int64_t record_rows,
                           const int32_t* __restrict__ page_table,
                           const int32_t* __restrict__ h2d, int32_t* __restrict__ physical) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t id = indices[i];
  int32_t out = -1;
  if (id >= 0 && id < history_end) {
    out = h2d[to_global(page_table, id)];
  } else if (transient_start >= 0 && id >= transient_start && id < written) {
    const int64_t row = slots + 1 + candidate_offset + id - transient_start;
    if (row < record_rows) out = (int32_t)row;
  }
  physical[i] = out;
}

struct Workspace {
  uint32_t* sel_bits;
  uint32_t* kept_bits;
  uint32_t* miss_bits;
  int32_t* word_offset;
  int64_t* misses;
  int64_t* chosen;
  uint64_t* keys;
  uint64_t* sorted;
  int64_t* counters;
  void* sort_temp;
  size_t sort_bytes;
  size_t total;
};

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

// The victim order sorts one key per pool slot on a few rank bits. rocPRIM
// takes its merge sort up to 2^20 keys (about 19 launches whatever the bit
// range); a merge-sort limit of 0 selects its onesweep radix sort, about one
// pass per 8 key bits.
using VictimSortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                    rocprim::default_config, 0>;

int plan(int64_t slots, int64_t history_capacity, uint8_t* base, Workspace* ws) {
  size_t sort_bytes = 0;
  hipError_t err = rocprim::radix_sort_keys<VictimSortConfig>(
      nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, (size_t)(slots + 1), 0,
      64, (hipStream_t)0, false);
  if (err != hipSuccess) {
    set_error("rocprim radix sort sizing failed: %s", hipGetErrorString(err));
    return kLaunchFailed;
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes);
    return base ? base + at : nullptr;
  };
  ws->sel_bits = reinterpret_cast<uint32_t*>(take(((history_capacity + 31) / 32) * 4));
  ws->kept_bits = reinterpret_cast<uint32_t*>(take(((slots + 1 + 31) / 32) * 4));
  ws->miss_bits = reinterpret_cast<uint32_t*>(take(((history_capacity + 31) / 32) * 4));
  ws->word_offset = reinterpret_cast<int32_t*>(take(((history_capacity + 31) / 32) * 4));
  ws->misses = reinterpret_cast<int64_t*>(take(history_capacity * 8));
  ws->chosen = reinterpret_cast<int64_t*>(take(history_capacity * 8));
  ws->keys = reinterpret_cast<uint64_t*>(take((slots + 1) * 8));
  ws->sorted = reinterpret_cast<uint64_t*>(take((slots + 1) * 8));
  ws->counters = reinterpret_cast<int64_t*>(take(kCounters * 8));
  ws->sort_temp = take(sort_bytes);
  ws->sort_bytes = sort_bytes;
  ws->total = off;
  return kOk;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_pool_workspace_bytes(int64_t slots, int64_t history_capacity, int64_t* bytes) {
  using namespace dsa;
  DSA_CHECK_ARG(slots >= 1 && history_capacity >= 0 && bytes, "invalid pool workspace query");
  Workspace ws{};
  int status = plan(slots, history_capacity, nullptr, &ws);
  if (status != kOk) return status;
  *bytes = (int64_t)ws.total;
  return kOk;
}

namespace dsa {
namespace {

// Orders `later` after the work enqueued so far on `earlier`, through one
// event per device. A wait captures the event's state when it is enqueued,
// so one event serves every call, provided no other thread records it between
// this call's record and wait: the lock is held across both.
int order_streams(hipStream_t earlier, hipStream_t later) {
  static std::mutex lock;
  static hipEvent_t events[64] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return kLaunchFailed;
  std::lock_guard<std::mutex> guard(lock);
  if (!events[device] && hipEventCreateWithFlags(&events[device], hipEventDisableTiming) != hipSuccess) {
    events[device] = nullptr;
    return kLaunchFailed;
  }
  if (hipEventRecord(events[device], earlier) != hipSuccess ||
      hipStreamWaitEvent(later, events[device], 0) != hipSuccess)
    return kLaunchFailed;
  return kOk;
}

// One recall on `stream` (the steps in the header). keep_floor >= 0 also
// keeps every slot stamped at or after it (a previous selection still being
// read on another stream); candidate ids map to the candidate rows from
// candidate_offset on. A gather_stream other than `stream` takes the gather
// of the missing records (after an event on `stream`), so that the next
// recall's bookkeeping on `stream` overlaps it; the caller gives that next
// recall another workspace and waits for the gather before reading the
// records.
int recall_impl(const int32_t* indices, int64_t n, const int32_t* page_table,
                int64_t history_end, int64_t written, int64_t transient_start,
                int64_t slots, const void* host, int64_t host_rows, void* records,
                int64_t record_rows, int64_t record_bytes, int32_t* h2d,
                int64_t* d2h, int64_t* priority, int64_t protect_stamp,
                int64_t chosen_stamp, void* workspace, int64_t workspace_bytes,
                int64_t history_capacity, int union_checked, int64_t* stats,
                int32_t* status, int32_t* physical, int64_t keep_floor,
                int64_t candidate_offset, hipStream_t stream, hipStream_t gather_stream) {
  DSA_CHECK_ARG(n >= 0 && slots >= 1 && history_end >= 0 && written >= history_end,
                "invalid recall shape");
  DSA_CHECK_ARG(history_end <= history_capacity, "history exceeds the planned workspace");
  DSA_CHECK_ARG(history_end < 0x7FFFFFFF, "history ids must fit int32");
  DSA_CHECK_ARG(history_end <= slots || union_checked,
                "recall without a host check needs history <= slots; otherwise the caller "
                "must have checked that the selection's union fits the pool");
  DSA_CHECK_ARG(record_rows >= slots + 1 && record_bytes > 0 && record_bytes % 16 == 0,
                "records must hold slots + 1 rows of a 16-byte multiple width");
  DSA_CHECK_ARG(transient_start < 0 || transient_start >= history_end,
                "the transient suffix starts after the host-backed history");
  DSA_CHECK_ARG(candidate_offset >= 0, "candidate offset must be nonnegative");
  DSA_CHECK_ARG(transient_start < 0 ||
                    written - transient_start + candidate_offset <= record_rows - (slots + 1),
                "transient suffix exceeds candidate slot capacity");
  DSA_CHECK_ARG(keep_floor < 0 || keep_floor < protect_stamp,
                "the keep floor must precede this recall's stamps");
  DSA_CHECK_ARG(protect_stamp >= 0 && chosen_stamp > protect_stamp && chosen_stamp < 0x7FFFFFFF,
                "invalid FIFO timestamps");
  DSA_CHECK_ARG(indices && page_table && h2d && d2h && priority && stats && physical && records &&
                    workspace,
                "null pointer");
  Workspace ws{};
  int rc = plan(slots, history_capacity, static_cast<uint8_t*>(workspace), &ws);
  if (rc != kOk) return rc;
  DSA_CHECK_ARG((int64_t)ws.total <= workspace_bytes, "workspace too small");
  void* mapped = nullptr;
  if (host_rows > 0) {
    hipError_t err = hipHostGetDevicePointer(&mapped, const_cast<void*>(host), 0);
    if (err != hipSuccess) {
      set_error("host records are not device-accessible pinned memory: %s",
                hipGetErrorString(err));
      return kInvalidArgument;
    }
  }
  const int64_t sel_words = (history_end + 31) / 32;
  const int64_t kept_words = (slots + 1 + 31) / 32;
  const int64_t clear_n = sel_words > kept_words ? sel_words : kept_words;
  hipLaunchKernelGGL(recall_clear, dim3((unsigned)((clear_n + 255) / 256 + 1)), dim3(256), 0,
                     stream, ws.sel_bits, sel_words, ws.kept_bits, kept_words, ws.counters);
  if (n > 0 && (history_end + 31) / 32 <= kMarkLdsWords)
    hipLaunchKernelGGL(recall_mark_lds, dim3((unsigned)((n + kMarkIdsPerBlock - 1) / kMarkIdsPerBlock)),
                       dim3(kMarkThreads), 0, stream, indices, n, history_end, written, ws.sel_bits,
                       status);
  else if (n > 0)
    hipLaunchKernelGGL(recall_mark, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       indices, n, history_end, written, ws.sel_bits, status);
  if (history_end > 0)
    hipLaunchKernelGGL(recall_lookup, dim3((unsigned)((history_end + 255) / 256)), dim3(256), 0,
                       stream, ws.sel_bits, history_end, page_table, h2d, priority, ws.kept_bits,
                       protect_stamp, ws.miss_bits);
  hipLaunchKernelGGL(recall_classify, dim3(1), dim3(kClassifyThreads), 0, stream, ws.sel_bits,
                     ws.miss_bits, history_end, ws.word_offset, ws.counters, stats);
  if (history_end > 0)
    hipLaunchKernelGGL(recall_emit, dim3((unsigned)((history_end + 255) / 256)), dim3(256), 0,
                       stream, ws.miss_bits, ws.word_offset, history_end, page_table, ws.misses);
  hipLaunchKernelGGL(recall_victim_keys, dim3((unsigned)((slots + 1 + 255) / 256)), dim3(256), 0,
                     stream, d2h, priority, ws.kept_bits, slots, keep_floor, ws.keys);
  // The keys arrive in slot order and the radix sort is stable, so sorting
  // only the rank bits (32 .. 32 + rank_bits) gives the (rank, slot) order of
  // a full 64-bit sort. Every stored priority is an earlier stamp, below
  // chosen_stamp, so rank + 1 <= chosen_stamp < 2^rank_bits - 1, the value
  // the kept slots' all-ones keys take in that range: they still sort last.
  // A few passes instead of eight.
  int rank_bits = 2;
  while (((int64_t)1 << (rank_bits - 1)) <= chosen_stamp) ++rank_bits;
  size_t sort_bytes = 0;
  hipError_t err = rocprim::radix_sort_keys<VictimSortConfig>(
      nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, (size_t)(slots + 1), 32,
      32 + rank_bits, stream, false);
  if (err == hipSuccess && sort_bytes > ws.sort_bytes) {
    set_error("rocprim radix sort needs %zu bytes of temporary storage, planned %zu",
              sort_bytes, ws.sort_bytes);
    return kLaunchFailed;
  }
  if (err == hipSuccess)
    err = rocprim::radix_sort_keys<VictimSortConfig>(ws.sort_temp, sort_bytes, ws.keys, ws.sorted,
                                                     (size_t)(slots + 1), 32, 32 + rank_bits,
                                                     stream, false);
  if (err != hipSuccess) {
    set_error("rocprim radix sort failed: %s", hipGetErrorString(err));
    return kLaunchFailed;
  }
  const int64_t assign_n = history_end > 0 ? history_end : 1;
  hipLaunchKernelGGL(recall_assign, dim3((unsigned)((assign_n + 255) / 256)), dim3(256), 0,
                     stream, ws.sorted, ws.misses, ws.counters, h2d, d2h, priority, chosen_stamp,
                     ws.chosen, stats, status);
  if (host_rows > 0) {
    // PCIe-bound: 128 work-groups (512 waves, one record each in flight)
    // keep the link at its rate (64 do not) and leave most CUs to the
    // kernels that overlap the copy.
    int64_t blocks = (history_end + 3) / 4;
    if (blocks > kGatherBlocks) blocks = kGatherBlocks;
    if (blocks < 1) blocks = 1;
    hipStream_t gs = stream;
    if (gather_stream != stream) {
      if (order_streams(stream, gather_stream) != kOk) {
        set_error("could not order the gather stream after the recall");
        return kLaunchFailed;
      }
      gs = gather_stream;
    }
    hipLaunchKernelGGL(recall_gather, dim3((unsigned)blocks), dim3(256), 0, gs,
                       static_cast<const uint8_t*>(mapped), static_cast<uint8_t*>(records),
                       ws.misses, ws.chosen, ws.counters, record_bytes);
  }
  if (n > 0)
    hipLaunchKernelGGL(recall_map, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       indices, n, history_end, written, transient_start, slots,
                       candidate_offset, record_rows, page_table, h2d, physical);
  DSA_CHECK_LAUNCH("exact recall");
  return kOk;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_pool_recall(const int32_t* indices, int64_t n, const int32_t* page_table,
                               int64_t history_end, int64_t written, int64_t transient_start,
                               int64_t slots, const void* host, int64_t host_rows, void* records,
                               int64_t record_rows, int64_t record_bytes, int32_t* h2d,
                               int64_t* d2h, int64_t* priority, int64_t protect_stamp,
                               int64_t chosen_stamp, void* workspace, int64_t workspace_bytes,
                               int64_t history_capacity, int union_checked, int64_t* stats,
                               int32_t* status, int32_t* physical, hipStream_t stream) {
  return dsa::recall_impl(indices, n, page_table, history_end, written, transient_start, slots, host,
                          host_rows, records, record_rows, record_bytes, h2d, d2h, priority,
                          protect_stamp, chosen_stamp, workspace, workspace_bytes,
                          history_capacity, union_checked, stats, status, physical, -1, 0, stream,
                          stream);
}

extern "C" int dsa_pool_recall_pipelined(
    const int32_t* indices, int64_t n, const int32_t* page_table, int64_t history_end,
    int64_t written, int64_t transient_start, int64_t slots, const void* host, int64_t host_rows,
    void* records, int64_t record_rows, int64_t record_bytes, int32_t* h2d, int64_t* d2h,
    int64_t* priority, int64_t protect_stamp, int64_t chosen_stamp, void* workspace,
    int64_t workspace_bytes, int64_t history_capacity, int union_checked, int64_t* stats,
    int32_t* status, int32_t* physical, int64_t keep_floor, int64_t candidate_offset,
    hipStream_t stream, hipStream_t gather_stream) {
  return dsa::recall_impl(indices, n, page_table, history_end, written, transient_start, slots, host,
                          host_rows, records, record_rows, record_bytes, h2d, d2h, priority,
                          protect_stamp, chosen_stamp, workspace, workspace_bytes,
                          history_capacity, union_checked, stats, status, physical, keep_floor,
                          candidate_offset, stream, gather_stream ? gather_stream : stream);
}

namespace dsa {
namespace {

// Release of a session's host rows from one layer's pool maps
// (cache/sparse_token_pool.py:697-710, release_ids): every host row of the
// session's pages that is resident frees its slot (d2h = MISSING, priority
// -1) and becomes MISSING in h2d. h2d and d2h are inverse on live entries, so
// no two threads touch the same slot.
__global__ void release_rows(const int32_t* __restrict__ page_table, int64_t pages,
                             int64_t host_rows, int32_t* __restrict__ h2d,
                             int64_t* __restrict__ d2h, int64_t* __restrict__ priority,
                             int64_t slots, int32_t* __restrict__ status) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= pages * kPage) return;
  const int64_t page = page_table[t / kPage];
  const int64_t row = page * kPage + t % kPage;
  if (page < 0 || row >= host_rows) {
    if (status) atomicOr(status, 1);
    return;
  }
  const int32_t slot = h2d[row];
  if (slot == kMissing) return;
  if (slot >= 1 && slot <= slots) {
    d2h[slot] = kMissing;
    priority[slot] = -1;
  } else if (status) {
    atomicOr(status, 1);
  }
  h2d[row] = kMissing;
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_pool_release_rows(const int32_t* page_table, int64_t pages, int64_t host_rows,
                                     int32_t* h2d, int64_t* d2h, int64_t* priority,
                                     int64_t slots, int32_t* status, hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(pages >= 0 && host_rows >= 0 && slots >= 1, "invalid release shape");
  if (pages == 0) return kOk;
  DSA_CHECK_ARG(pages * kPage < ((int64_t)1 << 40), "too many pages");
  DSA_CHECK_ARG(page_table && h2d && d2h && priority, "null pointer");
  const int64_t n = pages * kPage;
  hipLaunchKernelGGL(release_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     page_table, pages, host_rows, h2d, d2h, priority, slots, status);
  DSA_CHECK_LAUNCH("pool release");
  return kOk;
}
