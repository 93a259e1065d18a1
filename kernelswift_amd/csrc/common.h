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

// Two fp32 values to a packed bf16 pair (lo in bits 0-15) with the hardware conversion (v_cvt_pk_bf16_f32):
// RNE, subnormals kept, overflow to infinity; the same results as f32_to_bf16_rne for every non-NaN input.
typedef float cvt_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 cvt_bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((cvt_f32x2_t{lo, hi}), cvt_bf16x2_t));
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }


// ---------------------------------------------------------------- cross-lane exchange
// v_permlane16_swap / v_permlane32_swap (gfx950): the first operand's rows 1 and 3 (16-lane rows) trade
// places with the second operand's rows 0 and 2 (16_swap), or its rows 2-3 with the second's rows 0-1
// (32_swap).  Inline assembly: the builtin form was miscompiled when both operands carry the same value;
// the NOPs cover the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void permlane16_swap(uint32_t &a, uint32_t &b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(uint32_t &a, uint32_t &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// Value of lane (lane ^ S) for S in {1, 2, 4, 8, 16, 32}, without the LDS crossbar: DPP quad permutes,
// half-row mirror, row rotate, or a permlane swap.
// 16 bytes from global memory into LDS: lane i of the wave writes lds_base + 16 i (lds_base wave-uniform).
// Issued as inline assembly so that the compiler does not order the LDS reads of the other buffer behind
// it; completion is awaited explicitly (s_waitcnt vmcnt) before the barrier that publishes the data.
// base: wave-uniform 64-bit global address (SGPR pair), voff: per-lane byte offset, lds: LDS byte address.
__device__ __forceinline__ void dma16(const void *base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}

// LDS byte address of a __shared__ object (an address-space cast of a known LDS pointer, done once).
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T *p) {
  typedef __attribute__((address_space(3))) T lds_t;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_t *)(p)));
}

template <int S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  // (every lane's DPP source lies in its row, so the moves need no initial value)
  if constexpr (S == 1) {
    return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (S == 2) {
    return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (S == 4) {  // i ^ 4 = (i ^ 7) ^ 3: half-row mirror, then quad_perm [3,2,1,0]
    const uint32_t m = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);
    return __builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, false);
  } else if constexpr (S == 8) {
    return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (S == 16) {  // rows (0,1), (2,3) trade: even rows read the second result
    uint32_t a = x, b = x;
    permlane16_swap(a, b);
    return __builtin_amdgcn_inverse_ballot_w64(0xFFFF0000FFFF0000ull) ? a : b;
  } else {  // S == 32: rows (0,2), (1,3) trade
    uint32_t a = x, b = x;
    permlane32_swap(a, b);
    return __builtin_amdgcn_inverse_ballot_w64(0xFFFFFFFF00000000ull) ? a : b;
  }
}

// Maximum of x over the 64 lanes of a wave (every lane receives it), by lane_xor exchanges: no LDS round trips.
__device__ __forceinline__ float wave_max_f32(float x) {
  x = fmaxf(x, __builtin_bit_cast(float, lane_xor<32>(__builtin_bit_cast(uint32_t, x))));
  x = fmaxf(x, __builtin_bit_cast(float, lane_xor<16>(__builtin_bit_cast(uint32_t, x))));
  x = fmaxf(x, __builtin_bit_cast(float, lane_xor<8>(__builtin_bit_cast(uint32_t, x))));
  x = fmaxf(x, __builtin_bit_cast(float, lane_xor<4>(__builtin_bit_cast(uint32_t, x))));
  x = fmaxf(x, __builtin_bit_cast(float, lane_xor<2>(__builtin_bit_cast(uint32_t, x))));
  return fmaxf(x, __builtin_bit_cast(float, lane_xor<1>(__builtin_bit_cast(uint32_t, x))));
}

}  // namespace ks
