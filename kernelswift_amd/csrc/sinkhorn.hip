// Sinkhorn normalisation of 4x4 fp32 matrices (gfx950).
//
// Semantics: baseline/sinkhorn.py:13-19 —
//   x = softmax(x, -1) + eps; x /= colsum + eps; (repeat-1) x { x /= rowsum + eps; x /= colsum + eps }.
// The reference kernel (optimized/sinkhorn_project/op_kernel/sinkhorn_kernel.asc:168-189) keeps all
// iterations on chip; here every matrix lives in registers for the whole call.
//
// Two kernels, chosen by batch size (both read and write every byte exactly once):
// - fewer than 65536 matrices (latency-bound launches): lane g owns row (g % 4) of matrix (g / 4) as one
//   float4; row sums are in-lane, column sums are quad reductions with DPP quad permutes.  Four lanes per
//   matrix give four times the waves, which is what a short launch needs.
// - larger batches: one matrix per lane; global accesses stay fully coalesced through a per-wave LDS tile,
//   the matrix is carried as x_ij = a_i y_ij b_j so a normalisation step updates four scales instead of
//   rescaling sixteen elements, and persistent waves prefetch their next batch during the arithmetic.
// Reciprocals use v_rcp_f32 (<= 1 ulp) followed by a multiply; the result stays within a few fp32 ulps of
// true division after 20 normalisations (the reference needed a Newton step for its 10-bit reciprocal,
// optimized/sinkhorn_project/design.md:51-52).
#include "common.h"
#include "sinkhorn_quad.h"

namespace ks {
namespace {

__global__ __launch_bounds__(256) void sinkhorn4x4_kernel(const float4 *__restrict__ x, float4 *__restrict__ out,
                                                         int64_t n_rows, int repeat, float eps) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  // n_rows is a multiple of 4 and blocks are 256-aligned, so a quad is entirely live or entirely idle;
  // idle lanes still run the DPP exchanges on zeros (no divergence around cross-lane ops).
  const bool live = g < n_rows;
  float4 v = live ? x[g] : make_float4(0.f, 0.f, 0.f, 0.f);

  v = sinkhorn_quad_row(v, repeat, eps);
  if (live) out[g] = v;
}

// Matrix-per-lane form (large batches): lane t owns matrix t in 16 registers, so row and column sums
// are both in-lane and nothing is computed redundantly (the row-per-lane form recomputes every column sum
// and reciprocal in all four lanes of a quad).  Softmax uses v_exp_f32 and a reciprocal multiply.
// Global traffic stays fully coalesced: each wave loads a batch of 64 matrices (4 KiB) as four 1 KiB wave-wide
// rows of 16-byte chunks and passes them through a per-wave LDS tile to the matrix-per-lane layout (and
// back before the store).  In the tile, row r of matrix m sits at 16-byte unit 4m + (r ^ ((m >> 2) & 3)),
// which keeps both the coalesced-side and the matrix-side accesses of every 16 lanes on distinct banks.
// Waves are persistent (a grid of a few workgroups per CU) and walk batches with a stride; the next batch's four
// loads are issued before the current batch is computed, so every wave keeps 4 KiB in flight during its
// arithmetic instead of leaving the memory pipe idle between its load and compute phases (16M matrices:
// 4.7 -> 5.2 TB/s on the same box; the arithmetic and its results are unchanged).
constexpr int kSkWaves = 4;   // waves per block
constexpr int kSkBlocksPerCu = 12;

__device__ __forceinline__ int sk_unit(int m, int r) { return 4 * m + (r ^ ((m >> 2) & 3)); }

__global__ __launch_bounds__(64 * kSkWaves) void sinkhorn4x4_mat_kernel(const float4 *__restrict__ x,
                                                                       float4 *__restrict__ out, int64_t n_mats,
                                                                       int repeat, float eps) {
  __shared__ float4 tile[kSkWaves][256];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nb = (n_mats + 63) / 64;  // batches of 64 matrices
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSkWaves;
  float4 *T = tile[wave];
  // chunk c = 64 j + lane of batch bi is row c % 4 of matrix 64 bi + c / 4 (zeros past the last matrix)
  float4 nxt[4];
  auto load = [&](int64_t bi) {
    const int64_t chunks = 4 * (n_mats - 64 * bi);
    const float4 *src = x + 256 * bi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 64 * j + lane;
      nxt[j] = c < chunks ? src[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  int64_t bi = static_cast<int64_t>(blockIdx.x) * kSkWaves + wave;
  if (bi < nb) load(bi);
  for (; bi < nb; bi += stride) {  // uniform per wave (no block-wide synchronisation below)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 64 * j + lane;
      T[sk_unit(c >> 2, c & 3)] = nxt[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float v[16];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float4 a = T[sk_unit(lane, r)];
      v[4 * r] = a.x;
      v[4 * r + 1] = a.y;
      v[4 * r + 2] = a.z;
      v[4 * r + 3] = a.w;
    }
    if (bi + stride < nb) load(bi + stride);  // in flight during the arithmetic below
    // softmax over each row, then + eps (baseline/sinkhorn.py:14; no eps inside the softmax)
    constexpr float kLog2e = 1.44269504088896341f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float *w = v + 4 * r;
      const float ml = fmaxf(fmaxf(w[0], w[1]), fmaxf(w[2], w[3])) * kLog2e;
#pragma unroll
      for (int c = 0; c < 4; ++c) w[c] = __builtin_amdgcn_exp2f(__builtin_fmaf(w[c], kLog2e, -ml));
      const float q = rcp((w[0] + w[1]) + (w[2] + w[3]));
#pragma unroll
      for (int c = 0; c < 4; ++c) w[c] = __builtin_fmaf(w[c], q, eps);
    }
    // The matrix is kept as x_ij = a_i y_ij b_j with y the softmax output above: a row normalisation
    // divides a_i by (a_i sum_j y_ij b_j + eps) = (row sum + eps), a column normalisation b_j by
    // (b_j sum_i a_i y_ij + eps), so each step costs one 4-term dot and one reciprocal per row or column
    // instead of rescaling all 16 elements.
    float a[4] = {1.f, 1.f, 1.f, 1.f}, b[4] = {1.f, 1.f, 1.f, 1.f};
    auto col_step = [&]() {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float t = a[0] * v[c];
#pragma unroll
        for (int r = 1; r < 4; ++r) t = __builtin_fmaf(a[r], v[4 * r + c], t);
        b[c] *= rcp(__builtin_fmaf(b[c], t, eps));
      }
    };
    auto row_step = [&]() {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = v[4 * r] * b[0];
#pragma unroll
        for (int c = 1; c < 4; ++c) t = __builtin_fmaf(v[4 * r + c], b[c], t);
        a[r] *= rcp(__builtin_fmaf(a[r], t, eps));
      }
    };
    col_step();  // :15
    for (int it = 1; it < repeat; ++it) {  // :16-18
      row_step();
      col_step();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * r + c] = (a[r] * v[4 * r + c]) * b[c];
    // store through the tile (each lane rewrites only the units it read)
#pragma unroll
    for (int r = 0; r < 4; ++r) T[sk_unit(lane, r)] = make_float4(v[4 * r], v[4 * r + 1], v[4 * r + 2], v[4 * r + 3]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t chunks = 4 * (n_mats - 64 * bi);
    float4 *dst = out + 256 * bi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 64 * j + lane;
      if (c < chunks) dst[c] = T[sk_unit(c >> 2, c & 3)];
    }
    // the tile is rewritten by the next batch only after these reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
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
  if (n_mats < (int64_t(1) << 16)) {
    // small batches: one row per lane gives four times the waves, which is what a latency-bound launch needs
    const int64_t n_rows = n_mats * 4;
    hipLaunchKernelGGL(ks::sinkhorn4x4_kernel, dim3(static_cast<unsigned>(ks::ceil_div(n_rows, 256))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const float4 *>(x),
                       reinterpret_cast<float4 *>(out), n_rows, static_cast<int>(repeat), eps);
    KS_CHECK_LAUNCH("sinkhorn4x4_kernel");
    return KS_OK;
  }
  // persistent waves: a few workgroups per CU, each wave walking batches of 64 matrices
  int dev = 0, cus = 0;
  KS_CHECK_HIP(hipGetDevice(&dev));
  KS_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int64_t need = ks::ceil_div(ks::ceil_div(n_mats, 64), ks::kSkWaves);
  const int64_t cap = static_cast<int64_t>(cus > 0 ? cus : 1) * ks::kSkBlocksPerCu;
  const int64_t blocks = need < cap ? need : cap;
  hipLaunchKernelGGL(ks::sinkhorn4x4_mat_kernel, dim3(static_cast<unsigned>(blocks)), dim3(64 * ks::kSkWaves), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<const float4 *>(x),
                     reinterpret_cast<float4 *>(out), n_mats, static_cast<int>(repeat), eps);
  KS_CHECK_LAUNCH("sinkhorn4x4_mat_kernel");
  return KS_OK;
}
