// Shared helpers for the gfx950 DSA kernels: error reporting for the C ABI,
// wave64 shuffles, fp8-e4m3fn / bf16 conversions with exact rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

namespace dsa {

// ---------------------------------------------------------------- errors --
// Each C entry point returns 0 on success. On failure it returns a nonzero
// code and records a message retrievable with dsa_last_error(); the message
// is per host thread.
enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kLaunchFailed = 2,
  kUnsupported = 3,
};

void set_error(const char* fmt, ...);
void clear_error();

#define DSA_CHECK_ARG(cond, ...)            \
  do {                                      \
    if (!(cond)) {                          \
      ::dsa::set_error(__VA_ARGS__);        \
      return ::dsa::kInvalidArgument;       \
    }                                       \
  } while (0)

#define DSA_CHECK_LAUNCH(name)                                                  \
  do {                                                                          \
    hipError_t err_ = hipGetLastError();                                        \
    if (err_ != hipSuccess) {                                                   \
      ::dsa::set_error("%s launch failed: %s", name, hipGetErrorString(err_));  \
      return ::dsa::kLaunchFailed;                                              \
    }                                                                           \
  } while (0)

int device_cu_count();

// The exact top-k of the fused indexer step from the candidate lists that the
// logits kernel's candidate mode leaves (topk.hip; launched by logits.hip).
int topk_from_candidates(const uint8_t* q, const uint8_t* k, const float* weights,
                         const float* kscale, const int32_t* starts, const int32_t* ends,
                         int64_t query_start, const float* q_fold, float* scores, int64_t rows,
                         int64_t columns, int64_t ld, int64_t topk, float* values,
                         int32_t* indices, int64_t out_ld, const uint32_t* floors,
                         const uint32_t* records, const uint64_t* lists, int64_t splits,
                         int64_t per, int64_t cap, hipStream_t stream);

// ------------------------------------------------------------ numerics --
// fl32(1/448): the reciprocal the reference GPU path multiplies by.
constexpr float kReciprocal448 = 1.0f / 448.0f;
constexpr uint32_t kCanonicalNan = 0x7FFFFFFFu;

// float32 -> e4m3fn code, round to nearest even. Caller handles NaN; inputs
// are clamped to [-448, 448] so the overflow branch only catches NaN/inf.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float v) {
  uint32_t b = __float_as_uint(v);
  uint32_t sign = (b >> 24) & 0x80u;
  uint32_t a = b & 0x7FFFFFFFu;
  uint32_t code;
  if (a >= 0x43F00000u) {
    code = 0x7Fu;
  } else if (a < 0x3C800000u) {
    // Subnormal e4m3: m * 2^-9 with m in [0, 8]; m == 8 is code 0x08.
    code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    code = ((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
  }
  return code | sign;
}

// e4m3fn code -> float32 (exact). NaN code (S.1111.111) -> NaN.
__device__ __forceinline__ float e4m3fn_to_f32(uint32_t c) {
  uint32_t sign = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu;
  uint32_t m = c & 7u;
  float mag;
  if (e == 0) {
    mag = (float)m * 0.001953125f;  // 2^-9
  } else if (e == 15 && m == 7) {
    return __uint_as_float(sign | 0x7FC00000u);
  } else {
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

}  // namespace dsa
