// Shared host/device helpers for the gfx950 KernelSwift kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <string>

#include "../../include/kswift.h"

namespace ks {

// ---------------------------------------------------------------- errors
// Thread-local message of the last failing C-ABI call.
std::string &last_error();

// Format into last_error() and return `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

#define KS_CHECK_ARG(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::ks::fail(KS_ERR_INVALID, __VA_ARGS__);  \
  } while (0)

#define KS_CHECK_HIP(expr)                                                        \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess)                                                         \
      return ::ks::fail(KS_ERR_HIP, "%s failed: %s (%s:%d)", #expr,               \
                        hipGetErrorString(e_), __FILE__, __LINE__);               \
  } while (0)

// After a kernel launch: report launch-configuration errors.
#define KS_CHECK_LAUNCH(name)                                                     \
  do {                                                                            \
    hipError_t e_ = hipGetLastError();                                            \
    if (e_ != hipSuccess)                                                         \
      return ::ks::fail(KS_ERR_HIP, "launch of %s failed: %s", name,              \
                        hipGetErrorString(e_));                                   \
  } while (0)

inline bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// ---------------------------------------------------------------- bf16
// bf16 values travel as raw uint16_t bit patterns.
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (finite inputs; NaN kept quiet).
__host__ __device__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ks
