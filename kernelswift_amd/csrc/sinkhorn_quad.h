// Row-per-lane Sinkhorn of 4x4 fp32 matrices shared by the Sinkhorn kernel and the mHC mixing kernels:
// lane g of a quad owns row g % 4 as a float4; row sums are in-lane, column sums quad reductions with DPP
// quad permutes.  Semantics of baseline/sinkhorn.py:13-19 — x = softmax(x, -1) + eps; x /= colsum + eps;
// (repeat - 1) x { x /= rowsum + eps; x /= colsum + eps }.
#pragma once

#include "common.h"

namespace ks {
namespace {

// quad_perm encodings for DPP: [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E.
template <int CTRL>
__device__ __forceinline__ float dpp_quad(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 4 lanes of a quad; every lane receives the same value ((r0 + r1) + (r2 + r3)).
__device__ __forceinline__ float quad_sum(float v) {
  float a = v + dpp_quad<0xB1>(v);
  return a + dpp_quad<0x4E>(a);
}

__device__ __forceinline__ float rcp(float v) { return __builtin_amdgcn_rcpf(v); }

__device__ __forceinline__ void col_norm(float4 &v, float eps) {
  const float r0 = rcp(quad_sum(v.x) + eps);
  const float r1 = rcp(quad_sum(v.y) + eps);
  const float r2 = rcp(quad_sum(v.z) + eps);
  const float r3 = rcp(quad_sum(v.w) + eps);
  v.x *= r0;
  v.y *= r1;
  v.z *= r2;
  v.w *= r3;
}

__device__ __forceinline__ void row_norm(float4 &v, float eps) {
  const float r = rcp(((v.x + v.y) + (v.z + v.w)) + eps);
  v.x *= r;
  v.y *= r;
  v.z *= r;
  v.w *= r;
}

// One matrix row after the whole normalisation (every lane of the quad must be active: DPP exchanges).
__device__ __forceinline__ float4 sinkhorn_quad_row(float4 v, int repeat, float eps) {
  // softmax over the row, then + eps (baseline/sinkhorn.py:14; no eps inside the softmax)
  const float m = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
  const float e0 = expf(v.x - m), e1 = expf(v.y - m), e2 = expf(v.z - m), e3 = expf(v.w - m);
  const float s = (e0 + e1) + (e2 + e3);
  v.x = e0 / s + eps;
  v.y = e1 / s + eps;
  v.z = e2 / s + eps;
  v.w = e3 / s + eps;
  col_norm(v, eps);  // :15
  for (int it = 1; it < repeat; ++it) {  // :16-18
    row_norm(v, eps);
    col_norm(v, eps);
  }
  return v;
}

}  // namespace
}  // namespace ks
