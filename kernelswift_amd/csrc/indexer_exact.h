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

template <int CTRL>
__device__ __forceinline__ int64_t dpp_i64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u), CTRL, 0xF, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u >> 32), CTRL, 0xF, 0xF, false);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One product of bf16 values a, b (bit patterns) for the fixed-point accumulator below (bit i weighs
// 2^(i - 266)): false for a zero product, else v = hi 2^30 + lo (0 <= lo < 2^30) to be added at limbs li, li + 1.
__device__ __forceinline__ bool wide_product(uint32_t a, uint32_t b, int &li, int64_t &lo, int64_t &hi) {
  if ((a & 0x7FFFu) == 0u || (b & 0x7FFFu) == 0u) return false;
  const int ea = static_cast<int>((a >> 7) & 0xFFu), eb = static_cast<int>((b >> 7) & 0xFFu);
  const int64_t ma = static_cast<int64_t>((a & 0x7Fu) | (ea ? 0x80u : 0u));
  const int64_t mb = static_cast<int64_t>((b & 0x7Fu) | (eb ? 0x80u : 0u));
  const int o = (ea ? ea - 134 : -133) + (eb ? eb - 134 : -133) + 266;  // 0 .. 506
  li = o / 30;
  const int sh = o - 30 * li;
  const int64_t v = (((a ^ b) & 0x8000u) ? -(ma * mb) : ma * mb) * (int64_t(1) << sh);  // |v| < 2^46
  lo = v & 0x3FFFFFFF;
  hi = v >> 30;
  return true;
}

// The fixed-point sum held in 18 limbs of 30 bits (bit i weighs 2^(i - 266); limbs may carry any int64 value)
// rounded once to bf16 (RNE), +0 for an exact zero.
__device__ __forceinline__ uint16_t limbs_to_bf16(int64_t (&L)[18]) {
  constexpr int kNL = 18;
  auto normalize = [&]() {  // limbs 0..16 into [0, 2^30), the signed remainder in limb 17
#pragma unroll
    for (int i = 0; i + 1 < kNL; ++i) {
      const int64_t c = L[i] >> 30;
      L[i] -= c * (int64_t(1) << 30);
      L[i + 1] += c;
    }
  };
  normalize();
  const bool neg = L[kNL - 1] < 0;
  if (neg) {
#pragma unroll
    for (int i = 0; i < kNL; ++i) L[i] = -L[i];
    normalize();
  }
  int P = -1;  // position of the leading bit of the magnitude
#pragma unroll
  for (int i = kNL - 1; i >= 0; --i)
    if (P < 0 && L[i] != 0) P = 30 * i + 63 - __builtin_clzll(static_cast<uint64_t>(L[i]));
  if (P < 0) return 0;  // exact zero: +0
  const int lbit = P - 7 > 133 ? P - 7 : 133;  // the bf16 result's last bit (2^-133 is bit 133)
  const int s = lbit - 1, q = s / 30, r = s - 30 * q;  // rounding bit at bit r of limb q
  uint64_t lq = 0, lq1 = 0;
  bool sticky = false;
#pragma unroll
  for (int i = 0; i < kNL; ++i) {
    const uint64_t li = static_cast<uint64_t>(L[i]);
    lq = i == q ? li : lq;
    lq1 = i == q + 1 ? li : lq1;
    sticky = sticky || (i < q && li != 0u) || (i == q && (li & ((uint64_t(1) << r) - 1u)) != 0u);
  }
  const uint64_t w = (lq >> r) | (lq1 << (30 - r));  // bit 0: rounding bit; bits 1..8: the kept bits
  uint32_t kept = static_cast<uint32_t>(w >> 1) & 0x1FFu;
  if ((w & 1u) && (sticky || (kept & 1u))) ++kept;
  uint32_t bits = P - 7 >= 133 ? (static_cast<uint32_t>(P - 139) << 7) + kept - 128u : kept;
  if (bits >= 0x7F80u) bits = 0x7F80u;  // beyond the bf16 range: infinity
  return static_cast<uint16_t>((neg ? 0x8000u : 0u) | bits);
}

// Exact dot product of two bf16 rows of length KD, rounded once to bf16 (RNE), for rows of any dynamic
// range: a fixed-point integer accumulator whose bit i weighs 2^(i - 266).  Every bf16 value is m 2^l with
// |m| < 2^8 and l >= -133, so every product is an integer multiple of 2^-266 below 2^256, and the sum of
// 128 products stays below 2^540: 18 limbs of 30 bits, held in int64 so that carries can wait until the
// end.  The PARTS (2 or 4) adjacent lanes of a group each add the products of KD / PARTS consecutive
// elements (part = the lane's index in the group); DPP quad permutes sum the limbs.  qword(j) / kword(j)
// return elements 2j and 2j + 1 of the rows packed in a uint32.  Slow (every product touches the limbs
// through selects), and used only for dots whose spans exceed the double-precision paths.
template <int KD, int PARTS, class QW, class KW>
__device__ __attribute__((noinline)) uint16_t exact_dot_wide_bf16(QW qword, KW kword, int part) {
  static_assert(PARTS == 2 || PARTS == 4, "pairs or quads of lanes");
  constexpr int kNL = 18, kW = KD / 2 / PARTS;
  int64_t L[kNL];
#pragma unroll
  for (int i = 0; i < kNL; ++i) L[i] = 0;
#pragma unroll 1
  for (int j = part * kW; j < (part + 1) * kW; ++j) {
    const uint32_t qw = qword(j), kw = kword(j);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int li;
      int64_t lo, hi;
      if (!wide_product(h ? (qw >> 16) : (qw & 0xFFFFu), h ? (kw >> 16) : (kw & 0xFFFFu), li, lo, hi)) continue;
#pragma unroll
      for (int i = 0; i < kNL; ++i) L[i] += (i == li ? lo : 0) + (i == li + 1 ? hi : 0);
    }
  }
#pragma unroll
  for (int i = 0; i < kNL; ++i) {
    L[i] += dpp_i64<0xB1>(L[i]);                       // quad_perm [1, 0, 3, 2]: the pair
    if constexpr (PARTS == 4) L[i] += dpp_i64<0x4E>(L[i]);  // quad_perm [2, 3, 0, 1]: the other pair
  }
  return limbs_to_bf16(L);
}


// exact_dot_wide_bf16 of two rows of 128 elements computed by the whole wave, for kernels whose register budget
// cannot hold the limbs in every lane: lane l adds the products of elements 2l and 2l + 1 into 18 int64 limbs of
// wave-private LDS with 64-bit LDS atomics; the limbs are then read into wave-uniform values (scalar registers)
// and rounded by limbs_to_bf16.  qword(j) / kword(j): elements 2j and 2j + 1 packed in a uint32 (j = lane).
// Every lane of the wave must call it (the same dot); every lane receives the result.
template <class QW, class KW>
__device__ __forceinline__ uint16_t wave_exact_dot_wide_bf16(QW qword, KW kword, int64_t *limb) {
  const int lane = static_cast<int>(__lane_id());
  if (lane < 18) limb[lane] = 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t qw = qword(lane), kw = kword(lane);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int li;
    int64_t lo, hi;
    if (!wide_product(h ? (qw >> 16) : (qw & 0xFFFFu), h ? (kw >> 16) : (kw & 0xFFFFu), li, lo, hi)) continue;
    atomicAdd(reinterpret_cast<unsigned long long *>(&limb[li]), static_cast<unsigned long long>(lo));
    atomicAdd(reinterpret_cast<unsigned long long *>(&limb[li + 1]), static_cast<unsigned long long>(hi));
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint64_t mine = lane < 18 ? static_cast<uint64_t>(limb[lane]) : 0ull;
  int64_t L[18];
#pragma unroll
  for (int i = 0; i < 18; ++i) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(mine)), i));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(mine >> 32)), i));
    L[i] = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  }
  return limbs_to_bf16(L);
}

}  // namespace
}  // namespace ks
