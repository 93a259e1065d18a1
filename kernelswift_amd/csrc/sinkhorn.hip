// Sinkhorn normalisation of 4x4 fp32 matrices (gfx950).
//
// Semantics: baseline/sinkhorn.py:13-19 —
//   x = softmax(x, -1) + eps; x /= colsum + eps; (repeat-1) x { x /= rowsum + eps; x /= colsum + eps }.
// The reference kernel (optimized/sinkhorn_project/op_kernel/sinkhorn_kernel.asc:168-189) keeps all
// iterations on chip; here every matrix lives in registers for the whole call.
//
// Layout: matrix m is 16 contiguous floats (row-major); lane g owns row (g % 4) of matrix (g / 4) as one
// float4, so a wave moves 1 KiB of contiguous memory per load/store (fully coalesced 16-byte accesses).
// Row sums are in-lane; column sums are quad reductions with DPP quad permutes (no LDS, no barrier).
// Reciprocals use v_rcp_f32 (<= 1 ulp) followed by a multiply; the result stays within a few fp32 ulps of
// true division after 20 normalisations (the reference needed a Newton step for its 10-bit reciprocal,
// optimized/sinkhorn_project/design.md:51-52).
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

__global__ __launch_bounds__(256) void sinkhorn4x4_kernel(const float4 *__restrict__ x, float4 *__restrict__ out,
                                                         int64_t n_rows, int repeat, float eps) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  // n_rows is a multiple of 4 and blocks are 256-aligned, so a quad is entirely live or entirely idle;
  // idle lanes still run the DPP exchanges on zeros (no divergence around cross-lane ops).
  const bool live = g < n_rows;
  float4 v = live ? x[g] : make_float4(0.f, 0.f, 0.f, 0.f);

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
  if (live) out[g] = v;
}

}  // namespace
}  // namespace ks

extern "C" int ks_sinkhorn(const float *x, float *out, int64_t n_mats, int32_t repeat, float eps, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(n_mats >= 0 && n_mats < (int64_t(1) << 40), "ks_sinkhorn: n_mats=%lld out of range", (long long)n_mats);
  KS_CHECK_ARG(repeat >= 1, "ks_sinkhorn: repeat=%d must be >= 1", repeat);
  if (n_mats == 0) return KS_OK;
  KS_CHECK_ARG(x != nullptr && out != nullptr, "ks_sinkhorn: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16) && ks::aligned(out, 16), "ks_sinkhorn: x and out must be 16-byte aligned");
  const int64_t n_rows = n_mats * 4;
  const int64_t blocks = ks::ceil_div(n_rows, 256);
  hipLaunchKernelGGL(ks::sinkhorn4x4_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const float4 *>(x),
                     reinterpret_cast<float4 *>(out), n_rows, static_cast<int>(repeat), eps);
  KS_CHECK_LAUNCH("sinkhorn4x4_kernel");
  return KS_OK;
}
