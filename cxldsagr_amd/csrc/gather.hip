// A11: top-k-driven gather of fixed-width records from pinned host DRAM into
// HBM, read by the GPU over PCIe (zero-copy), plus a contiguous H2D copy.
//
// Semantics: operators/common/kv_transfer.py:21-103 and
// operators/common/csrc/kv_transfer.cu:14-99 - device[device_ids[r]] =
// host[host_ids[r]] for r < valid_count (or all r), whole records, 16-byte
// vector copies when both rows and the width allow it, bytes otherwise.
//
// Differences by design: the reference traps on an out-of-range id; a GPU
// trap is not acceptable here, so an invalid id (or a valid_count outside
// [0, count]) skips the row and ORs a bit into the caller's status word
// (1 = id out of range, 2 = bad count), which the host checks when it wants.
//
// Mapping: one wave per record (a 656-byte fp8 record is 41 x 16 B, a
// 1152-byte bf16 record 72 x 16 B), grid-stride over records, so many PCIe
// reads are in flight at once.
#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;

template <typename CountT>
__global__ __launch_bounds__(kThreads) void gather_records(
    const uint8_t* __restrict__ host, uint8_t* __restrict__ device,
    const int64_t* __restrict__ host_ids, const int64_t* __restrict__ device_ids, int64_t count,
    int64_t host_rows, int64_t device_rows, int64_t row_bytes, const CountT* __restrict__ valid,
    int32_t* __restrict__ status) {
  int64_t active = count;
  if (valid != nullptr) {
    const int64_t v = (int64_t)*valid;
    if (v < 0 || v > count) {
      if (blockIdx.x == 0 && threadIdx.x == 0 && status) atomicOr(status, 2);
      return;
    }
    active = v;
  }
  const int lane = threadIdx.x & 63;
  const int64_t first = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t r = first; r < active; r += stride) {
    const int64_t h = host_ids[r];
    const int64_t d = device_ids[r];
    if (h < 0 || h >= host_rows || d < 0 || d >= device_rows) {
      if (lane == 0 && status) atomicOr(status, 1);
      continue;
    }
    const uint8_t* src = host + h * row_bytes;
    uint8_t* dst = device + d * row_bytes;
    if ((row_bytes & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
      const int64_t n = row_bytes >> 4;
      for (int64_t i = lane; i < n; i += 64)
        reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    } else {
      for (int64_t i = lane; i < row_bytes; i += 64) dst[i] = src[i];
    }
  }
}

}  // namespace
}  // namespace dsa

extern "C" int dsa_gather_records(const void* host, int64_t host_rows, void* device,
                                  int64_t device_rows, int64_t row_bytes,
                                  const int64_t* host_ids, const int64_t* device_ids,
                                  int64_t count, const void* valid_count, int count_kind,
                                  int64_t max_blocks, int32_t* status, hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(count >= 0 && host_rows >= 0 && device_rows >= 0 && row_bytes > 0,
                "invalid record gather shape");
  DSA_CHECK_ARG(max_blocks >= 0 && max_blocks < 0x7FFFFFFF, "max_ctas must be a positive grid size");
  DSA_CHECK_ARG(valid_count == nullptr || count_kind == DSA_COUNT_I64 || count_kind == DSA_COUNT_U32,
                "valid_count must be int64 or uint32");
  if (count == 0) return kOk;
  DSA_CHECK_ARG(host && device && host_ids && device_ids, "null pointer");
  void* mapped = nullptr;
  hipError_t err = hipHostGetDevicePointer(&mapped, const_cast<void*>(host), 0);
  if (err != hipSuccess) {
    set_error("host records are not device-accessible pinned memory: %s", hipGetErrorString(err));
    return kInvalidArgument;
  }
  int64_t blocks = (count + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t cap = max_blocks ? max_blocks : 4096;
  if (blocks > cap) blocks = cap;
  const uint8_t* src = static_cast<const uint8_t*>(mapped);
  uint8_t* dst = static_cast<uint8_t*>(device);
  if (valid_count == nullptr || count_kind == DSA_COUNT_I64)
    hipLaunchKernelGGL(gather_records<int64_t>, dim3((unsigned)blocks), dim3(kThreads), 0, stream,
                       src, dst, host_ids, device_ids, count, host_rows, device_rows, row_bytes,
                       static_cast<const int64_t*>(valid_count), status);
  else
    hipLaunchKernelGGL(gather_records<uint32_t>, dim3((unsigned)blocks), dim3(kThreads), 0, stream,
                       src, dst, host_ids, device_ids, count, host_rows, device_rows, row_bytes,
                       static_cast<const uint32_t*>(valid_count), status);
  DSA_CHECK_LAUNCH("record gather");
  return kOk;
}

extern "C" int dsa_copy_records_h2d(const void* host, void* device, int64_t bytes,
                                    hipStream_t stream) {
  using namespace dsa;
  DSA_CHECK_ARG(bytes >= 0, "byte count must be nonnegative");
  if (bytes == 0) return kOk;
  DSA_CHECK_ARG(host && device, "null pointer");
  hipError_t err = hipMemcpyAsync(device, host, (size_t)bytes, hipMemcpyHostToDevice, stream);
  if (err != hipSuccess) {
    set_error("hipMemcpyAsync failed: %s", hipGetErrorString(err));
    return kLaunchFailed;
  }
  return kOk;
}
