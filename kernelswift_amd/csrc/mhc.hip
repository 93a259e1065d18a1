// Manifold-constrained hyper-connection (mHC) mixing with the Sinkhorn normalisation fused in (gfx950).
//
// The reference configures the DeepSeek residual hyper-connections (hc_mult = 4 streams,
// hc_sinkhorn_iters = 20, hc_eps; baseline/indexer.py:48-50) and ships their 4x4 Sinkhorn projection as
// an operator of its own (baseline/sinkhorn.py; mhc = 4 there).  A layer with hc_mult = n keeps n residual
// streams x[t] in R^{n x C} per token; from logits computed on the flattened, normalised streams it forms
//   H_pre  = sigmoid(pre logits)        (n)       the layer input   h = H_pre x            (ks_mhc_pre)
//   H_post = 2 sigmoid(post logits)     (n)       the residual update
//   H_res  = Sinkhorn(res logits)       (n x n)   x' = H_res x + H_post^T f(h)            (ks_mhc_post)
// with the Sinkhorn of baseline/sinkhorn.py:13-19 (softmax + eps, column pass, then repeat - 1 row /
// column passes).  Here the Sinkhorn runs inside its consumer: ks_mhc_post normalises each token's 4x4
// logits in registers (a quad of lanes, one row per lane) and applies the doubly stochastic matrix to the
// streams in the same pass, so the matrices never reach memory and no Sinkhorn launch is needed.
//
// Work decomposition (both kernels HBM-bound streams): one wave per token; every quad of the wave
// computes the token's matrix (the DPP reductions keep the quads independent), lanes then gather the four
// rows by quad broadcasts, and the wave streams the token's columns in 16-byte chunks (8 bf16) with fully
// coalesced loads of the n stream rows and of f, fp32 arithmetic, and RNE bf16 stores.
#include "common.h"
#include "sinkhorn_quad.h"

namespace ks {
namespace {

constexpr int kMhcWaves = 4;  // tokens (waves) per workgroup
constexpr int kMhcN = 4;      // hc_mult

// Value of lane (lane & ~3) + SRC of the quad (DPP quad_perm [SRC, SRC, SRC, SRC]).
template <int SRC>
__device__ __forceinline__ float quad_bcast(float v) {
  constexpr int ctrl = SRC | (SRC << 2) | (SRC << 4) | (SRC << 6);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + expf(-z)); }

__device__ __forceinline__ void unpack8(uint4 u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    v[2 * p] = bf16_to_f32(static_cast<uint16_t>(w[p] & 0xFFFFu));
    v[2 * p + 1] = bf16_to_f32(static_cast<uint16_t>(w[p] >> 16));
  }
}

__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p)
    w[p] = cvt_pk_bf16(v[2 * p], v[2 * p + 1]);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// out[t, i, :] = sum_j H_res[t][i][j] x[t, j, :] + H_post[t][i] f[t, :]   (out may alias x: each lane reads
// its columns of all four streams before writing them)
__global__ __launch_bounds__(64 * kMhcWaves) void mhc_post_kernel(const uint16_t *x, const uint16_t *__restrict__ f,
                                                                 const float *__restrict__ res_logits,
                                                                 const float *__restrict__ post_logits, uint16_t *out,
                                                                 int64_t N, int64_t C8, int repeat, float eps) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kMhcWaves + wave;
  if (t >= N) return;  // uniform per wave
  const int r = lane & 3;
  // the token's Sinkhorn: lane r of every quad normalises row r (all lanes active for the DPP exchanges)
  float4 row = reinterpret_cast<const float4 *>(res_logits + t * 16)[r];
  const float4 pl = reinterpret_cast<const float4 *>(post_logits + t * 4)[0];
  row = sinkhorn_quad_row(row, repeat, eps);
  float M[kMhcN][kMhcN];
  {
    const float rc[4] = {row.x, row.y, row.z, row.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      M[0][j] = quad_bcast<0>(rc[j]);
      M[1][j] = quad_bcast<1>(rc[j]);
      M[2][j] = quad_bcast<2>(rc[j]);
      M[3][j] = quad_bcast<3>(rc[j]);
    }
  }
  const float p[4] = {2.f * sigmoid(pl.x), 2.f * sigmoid(pl.y), 2.f * sigmoid(pl.z), 2.f * sigmoid(pl.w)};
  const int64_t C = C8 * 8;
  const uint4 *xs = reinterpret_cast<const uint4 *>(x + t * kMhcN * C);
  const uint4 *fs = reinterpret_cast<const uint4 *>(f + t * C);
  uint4 *os = reinterpret_cast<uint4 *>(out + t * kMhcN * C);
  for (int64_t c = lane; c < C8; c += 64) {
    uint4 xu[kMhcN];
#pragma unroll
    for (int j = 0; j < kMhcN; ++j) xu[j] = xs[j * C8 + c];
    const uint4 fu = fs[c];
    float xv[kMhcN][8], fv[8];
#pragma unroll
    for (int j = 0; j < kMhcN; ++j) unpack8(xu[j], xv[j]);
    unpack8(fu, fv);
#pragma unroll
    for (int i = 0; i < kMhcN; ++i) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = M[i][0] * xv[0][e];
        acc = __builtin_fmaf(M[i][1], xv[1][e], acc);
        acc = __builtin_fmaf(M[i][2], xv[2][e], acc);
        acc = __builtin_fmaf(M[i][3], xv[3][e], acc);
        o[e] = __builtin_fmaf(p[i], fv[e], acc);
      }
      os[i * C8 + c] = pack8(o);
    }
  }
}

// h[t, :] = sum_j sigmoid(pre_logits[t][j]) x[t, j, :]
__global__ __launch_bounds__(64 * kMhcWaves) void mhc_pre_kernel(const uint16_t *__restrict__ x,
                                                                const float *__restrict__ pre_logits,
                                                                uint16_t *__restrict__ h, int64_t N, int64_t C8) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kMhcWaves + wave;
  if (t >= N) return;
  const float4 pl = reinterpret_cast<const float4 *>(pre_logits + t * 4)[0];
  const float g[4] = {sigmoid(pl.x), sigmoid(pl.y), sigmoid(pl.z), sigmoid(pl.w)};
  const uint4 *xs = reinterpret_cast<const uint4 *>(x + t * kMhcN * C8 * 8);
  uint4 *hs = reinterpret_cast<uint4 *>(h + t * C8 * 8);
  for (int64_t c = lane; c < C8; c += 64) {
    uint4 xu[kMhcN];
#pragma unroll
    for (int j = 0; j < kMhcN; ++j) xu[j] = xs[j * C8 + c];
    float xv[kMhcN][8], o[8];
#pragma unroll
    for (int j = 0; j < kMhcN; ++j) unpack8(xu[j], xv[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = g[0] * xv[0][e];
      acc = __builtin_fmaf(g[1], xv[1][e], acc);
      acc = __builtin_fmaf(g[2], xv[2][e], acc);
      o[e] = __builtin_fmaf(g[3], xv[3][e], acc);
    }
    hs[c] = pack8(o);
  }
}

int check_mhc(const void *x, int64_t N, int64_t C, const char *what) {
  KS_CHECK_ARG(N >= 0 && N < (int64_t(1) << 31), "%s: N=%lld out of range", what, (long long)N);
  KS_CHECK_ARG(C >= 8 && C % 8 == 0, "%s: C=%lld must be a positive multiple of 8", what, (long long)C);
  KS_CHECK_ARG(N == 0 || x != nullptr, "%s: null pointer", what);
  return KS_OK;
}

}  // namespace
}  // namespace ks

extern "C" int ks_mhc_pre(const uint16_t *x, const float *pre_logits, uint16_t *h, int64_t N, int64_t C,
                          void *stream) {
  ks::last_error().clear();
  int rc = ks::check_mhc(x, N, C, "ks_mhc_pre");
  if (rc != KS_OK) return rc;
  if (N == 0) return KS_OK;
  KS_CHECK_ARG(pre_logits && h, "ks_mhc_pre: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16) && ks::aligned(h, 16) && ks::aligned(pre_logits, 16),
               "ks_mhc_pre: x and h must be 16-byte aligned, pre_logits 16-byte aligned");
  hipLaunchKernelGGL(ks::mhc_pre_kernel, dim3(static_cast<unsigned>(ks::ceil_div(N, ks::kMhcWaves))),
                     dim3(64 * ks::kMhcWaves), 0, static_cast<hipStream_t>(stream), x, pre_logits, h, N, C / 8);
  KS_CHECK_LAUNCH("mhc_pre_kernel");
  return KS_OK;
}

extern "C" int ks_mhc_post(const uint16_t *x, const uint16_t *f, const float *res_logits, const float *post_logits,
                           uint16_t *out, int64_t N, int64_t C, int32_t sinkhorn_iters, float eps, void *stream) {
  ks::last_error().clear();
  int rc = ks::check_mhc(x, N, C, "ks_mhc_post");
  if (rc != KS_OK) return rc;
  KS_CHECK_ARG(sinkhorn_iters >= 1, "ks_mhc_post: sinkhorn_iters must be >= 1");
  if (N == 0) return KS_OK;
  KS_CHECK_ARG(f && res_logits && post_logits && out, "ks_mhc_post: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16) && ks::aligned(f, 16) && ks::aligned(out, 16) && ks::aligned(res_logits, 16) &&
                   ks::aligned(post_logits, 16),
               "ks_mhc_post: every buffer must be 16-byte aligned");
  hipLaunchKernelGGL(ks::mhc_post_kernel, dim3(static_cast<unsigned>(ks::ceil_div(N, ks::kMhcWaves))),
                     dim3(64 * ks::kMhcWaves), 0, static_cast<hipStream_t>(stream), x, f, res_logits, post_logits, out,
                     N, C / 8, static_cast<int>(sinkhorn_iters), eps);
  KS_CHECK_LAUNCH("mhc_post_kernel");
  return KS_OK;
}
