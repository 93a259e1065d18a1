// Declarations shared by the indexer kernels (RoPE/statistics, scores, top-k, fused entry).
#pragma once

#include "common.h"

namespace ks {

// Exponent of the least significant bit of a nonzero bf16 value: value = m * 2^lsb, m integer.
__host__ __device__ inline int bf16_lsb_exponent(uint16_t b) {
  const int e = (b >> 7) & 0xFF;
  return e == 0 ? -133 : e - 134;
}

// MFMA accumulation error model used by the score kernel: |fp32 MFMA dot - exact dot| is assumed
// below kScoreBoundC * 2^-23 * ||q|| * ||k||.  Measured maximum on gfx950 for D = 128:
// 0.68 (N(0,1) data) and 1.52 (heavy-tailed x^3 data) in the same units; 3.0 leaves >= 2x margin.
constexpr float kScoreBoundC = 3.0f;

int launch_rope_rows(const uint16_t *src, uint16_t *dst, const float *freqs, int64_t rows, int D, int H, int64_t S,
                     int64_t pos0, int rope_start, int rope_dim, float *norm, int32_t *span, hipStream_t stream);

int launch_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                          const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B,
                          int64_t S, int64_t H, int64_t D, int64_t T, int64_t kbs, int causal, int64_t start_pos,
                          int ratio, float bound_c, uint32_t *stats, hipStream_t stream);

}  // namespace ks
