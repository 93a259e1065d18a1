// Exact-score arithmetic shared by the indexer score kernel and the top-k kernel's exact recomputation of
// candidate scores (gfx950): MFMA tile, interval-test conversion, exact bf16 rounding of double-precision
// dot products, and the canonical combination of the four head-group sums.
#pragma once

#include "common.h"
#include "indexer_common.h"

namespace ks {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ float round_bf16_f(float a) { return bf16_to_f32(f32_to_bf16_rne(a)); }

// Packed RNE conversion of two fp32 values and ReLU on the bf16 bit patterns (negative bf16 values are
// negative int16, so a signed max with 0 clears them to +0).
__device__ __forceinline__ uint32_t cvt_relu_pk(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t);  // one v_cvt_pk_bf16_f32
  const short2_t s = __builtin_elementwise_max(__builtin_bit_cast(short2_t, v), short2_t{0, 0});
  return __builtin_bit_cast(uint32_t, s);
}

__device__ __forceinline__ float unpack_hi(uint32_t p) { return __builtin_bit_cast(float, p & 0xFFFF0000u); }
__device__ __forceinline__ float unpack_lo(uint32_t p) { return __builtin_bit_cast(float, p << 16); }

__device__ __forceinline__ int frexp_exp(float x) {
  int e = 0;
  frexpf(x, &e);
  return e;
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u), CTRL, 0xF, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Sum over the 4 lanes of a quad (quad_perm xor 1, xor 2); exact whenever every partial sum is.
__device__ __forceinline__ double quad_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);
  return v + dpp_f64<0x4E>(v);
}

// RNE to bf16 of a double value s, with the sign of a residual t (s + t is the exact value, |t| below the
// double spacing at s) deciding exact bf16 midpoints; t == 0 ties to even.
__device__ uint16_t round_dir_to_bf16(double s, int tdir) {
  if (s == 0.0) return 0;
  const uint64_t bits = __builtin_bit_cast(uint64_t, s);
  const uint16_t sign = (bits >> 63) ? 0x8000 : 0;
  const uint64_t mag = bits & 0x7FFFFFFFFFFFFFFFull;
  const int e = static_cast<int>(mag >> 52) - 1023;
  if (e >= -126) {
    uint64_t kept = mag >> 45;
    const uint64_t rem = mag & ((1ull << 45) - 1);
    const uint64_t half = 1ull << 44;
    const bool up = rem > half || (rem == half && (tdir > 0 || (tdir == 0 && (kept & 1))));
    if (up) ++kept;
    const int ebf = static_cast<int>(kept >> 7) - 1023 + 127;
    if (ebf >= 255) return sign | 0x7F80;
    return sign | static_cast<uint16_t>(ebf << 7) | static_cast<uint16_t>(kept & 0x7F);
  }
  const double x = ldexp(fabs(s), 133);  // exact; x < 2^7
  const double n = floor(x);
  const double rem = x - n;
  const uint32_t ni = static_cast<uint32_t>(n);
  const bool up = rem > 0.5 || (rem == 0.5 && (tdir > 0 || (tdir == 0 && (ni & 1))));
  return sign | static_cast<uint16_t>(ni + (up ? 1u : 0u));  // 128 -> smallest normal, bits 0x0080
}

// RNE to bf16 of the exact value a + b (two doubles): TwoSum gives s + t == a + b exactly.
__device__ uint16_t round2_to_bf16(double a, double b) {
  const double s = a + b;
  const double bb = s - a;
  const double t = (a - (s - bb)) + (b - bb);
  return round_dir_to_bf16(s, (t == 0.0) ? 0 : (((t > 0.0) == (s > 0.0)) ? 1 : -1));
}

// RNE to bf16 of a double s with |s| in [2^-126, 2^127) (or s == 0): round to fp32 with round-to-odd (the
// RNE conversion, stepped one unit toward zero when it went away from zero, with the last bit set when it
// was inexact), then RNE to bf16.  Rounding to odd at 24 bits and then to nearest at 8 bits equals direct
// rounding to nearest at 8 bits (the intermediate keeps more than two extra bits).
__device__ __forceinline__ uint16_t round_to_bf16_fast(double s) {
  const float f = static_cast<float>(s);
  const double back = static_cast<double>(f);
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if (back != s) u = (u - (fabs(back) > fabs(s) ? 1u : 0u)) | 1u;
  return f32_to_bf16_rne(__builtin_bit_cast(float, u));
}

// ((G0 + G1) + (G2 + G3)) over the four 16-lane rows of the wave (row g holds head group g), returned in
// every lane.  v_permlane16_swap exchanges row 1 of its first operand with row 0 of its second (and rows
// 3 / 2), so with G in both operands every lane ends up holding its row pair's two values; the sum of the
// two registers is G0 + G1 in rows 0-1 and G2 + G3 in rows 2-3.  v_permlane32_swap does the same across
// the wave halves.  Written as inline assembly (the builtin form was miscompiled into v + v when both
// operands carry the same value); the NOPs cover the VALU-write -> permlane-read hazard.
__device__ __forceinline__ float combine_groups(float G) {
  float a = G, b = G;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  float c = a + b, d = c;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(c), "+v"(d));
  return c + d;
}

// bf16 value >= |w| (|w| rounded toward +inf to bf16), for bounds that must not underestimate.
__device__ __forceinline__ uint16_t bf16_abs_round_up(float w) {
  const uint32_t u = __builtin_bit_cast(uint32_t, w) & 0x7FFFFFFFu;
  return static_cast<uint16_t>((u + 0xFFFFu) >> 16);
}

// Exact dot product of two bf16 rows of length KD rounded once to bf16 (RNE), computed by a quad of lanes:
// lane quarter `sub` multiplies elements KD/4 sub .. KD/4 (sub + 1) - 1 in double precision, and a DPP
// quad reduction adds the quarters.  span_sum = span(q row) + span(k row) (row statistics) proves the
// path exact: every partial sum is a multiple of the smallest product LSB and stays below 2^53 of it when
// span_sum <= 52 (plain double sums); up to 84 the products above / below 2^(top - 38) accumulate
// separately (top = exponent of norm_q * norm_k), each exactly, and one TwoSum-based rounding combines
// them.  Beyond 84 the result is not exact: `exact` is cleared and the lower interval end is the caller's
// choice.  FAST (wave-uniform): every quad of the wave has span_sum <= 52.
template <int KD>
__device__ uint16_t exact_dot_bf16(const uint16_t *__restrict__ qrow, const uint16_t *__restrict__ krow, int sub,
                                   int span_sum, float qnorm, float knorm, bool fast, bool &exact) {
  constexpr int kLC = KD / 32;  // 16-byte chunks per lane
  exact = span_sum <= 84;
  if (fast) {
    const uint4 *qp = reinterpret_cast<const uint4 *>(qrow + (KD / 4) * sub);
    const uint4 *kp = reinterpret_cast<const uint4 *>(krow + (KD / 4) * sub);
    uint4 qc[kLC], kc[kLC];
#pragma unroll
    for (int c = 0; c < kLC; ++c) {
      qc[c] = qp[c];
      kc[c] = kp[c];
    }
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int c = 0; c < kLC; ++c) {
      const uint32_t qw[4] = {qc[c].x, qc[c].y, qc[c].z, qc[c].w};
      const uint32_t kw[4] = {kc[c].x, kc[c].y, kc[c].z, kc[c].w};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        a0 = __builtin_fma(static_cast<double>(unpack_lo(qw[p])), static_cast<double>(unpack_lo(kw[p])), a0);
        a1 = __builtin_fma(static_cast<double>(unpack_hi(qw[p])), static_cast<double>(unpack_hi(kw[p])), a1);
      }
    }
    const double sum = quad_sum_f64(a0 + a1);
    const bool outside = sum != 0.0 && !(fabs(sum) >= 0x1p-126 && fabs(sum) < 0x1p127);
    if (__builtin_amdgcn_ballot_w64(outside) == 0ull) return round_to_bf16_fast(sum);
    return round_dir_to_bf16(sum, 0);
  }
  const int top_sum = frexp_exp(qnorm) + frexp_exp(knorm);
  const bool split = span_sum > 52;
  const double thr = split ? ldexp(1.0, top_sum - 38) : 0.0;
  double hi = 0.0, lo = 0.0;
  const uint32_t *q32 = reinterpret_cast<const uint32_t *>(qrow + (KD / 4) * sub);
  const uint32_t *k32 = reinterpret_cast<const uint32_t *>(krow + (KD / 4) * sub);
#pragma unroll 1
  for (int j = 0; j < KD / 8; ++j) {
    const uint32_t qw = q32[j], kw = k32[j];
    const double p0 = static_cast<double>(unpack_lo(qw)) * static_cast<double>(unpack_lo(kw));
    const double p1 = static_cast<double>(unpack_hi(qw)) * static_cast<double>(unpack_hi(kw));
    if (!split || fabs(p0) >= thr) hi += p0; else lo += p0;
    if (!split || fabs(p1) >= thr) hi += p1; else lo += p1;
  }
  return round2_to_bf16(quad_sum_f64(hi), quad_sum_f64(lo));
}

}  // namespace
}  // namespace ks
