// Diagnostic export: chains of v_mfma_f32_16x16x32_bf16 on caller-given operands.
//
// The indexer's exactness argument bounds the difference between the MFMA's fp32 result and the exact dot
// product with a model of how one MFMA accumulates (exact products, a sum of the 32 products and the
// accumulator, one rounding of the result).  This entry runs the instruction exactly as the score kernels
// do, on operands chosen by a test, so that the model is checked on the hardware the library runs on.
//
// Layout per test t (one wave each):
//   a  bf16 [t][nchain][16 rows][32 k]      (row-major A operands of the chained MFMAs)
//   bt bf16 [t][nchain][16 cols][32 k]      (B operands, stored column by column)
//   c  f32  [t][16][16], d f32 [t][16][16]  d = chain of d_j = a_j . b_j + d_{j-1}, d_{-1} = c
// Lane l holds A row l % 16, k = 8 (l / 16) .. + 7, B column l % 16, same k, and D rows 4 (l / 16) + i.
#include "common.h"
#include "indexer_exact.h"

namespace ks {
namespace {

__global__ __launch_bounds__(64) void mfma_chain_kernel(const uint16_t *__restrict__ a, const uint16_t *__restrict__ bt,
                                                       const float *__restrict__ c, float *__restrict__ d,
                                                       int nchain) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  f32x4_t acc;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = c[t * 256 + (4 * g + i) * 16 + r];
  for (int j = 0; j < nchain; ++j) {
    const int64_t base = (t * nchain + j) * 512;
    const uint4 av = *reinterpret_cast<const uint4 *>(a + base + r * 32 + 8 * g);
    const uint4 bv = *reinterpret_cast<const uint4 *>(bt + base + r * 32 + 8 * g);
    acc = mfma16(av, bv, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) d[t * 256 + (4 * g + i) * 16 + r] = acc[i];
}

}  // namespace
}  // namespace ks

// Not part of the public header (a test instrument).  ntests >= 0, 1 <= nchain <= 64.
extern "C" int ks_dbg_mfma_bf16_chain(const uint16_t *a, const uint16_t *bt, const float *c, float *d, int64_t ntests,
                                      int32_t nchain, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(ntests >= 0 && ntests < (int64_t(1) << 31), "ks_dbg_mfma_bf16_chain: ntests out of range");
  KS_CHECK_ARG(nchain >= 1 && nchain <= 64, "ks_dbg_mfma_bf16_chain: nchain must be in [1, 64]");
  if (ntests == 0) return KS_OK;
  KS_CHECK_ARG(a && bt && c && d, "ks_dbg_mfma_bf16_chain: null pointer");
  KS_CHECK_ARG(ks::aligned(a, 16) && ks::aligned(bt, 16), "ks_dbg_mfma_bf16_chain: operands must be 16-byte aligned");
  hipLaunchKernelGGL(ks::mfma_chain_kernel, dim3(static_cast<unsigned>(ntests)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), a, bt, c, d, static_cast<int>(nchain));
  KS_CHECK_LAUNCH("mfma_chain_kernel");
  return KS_OK;
}
