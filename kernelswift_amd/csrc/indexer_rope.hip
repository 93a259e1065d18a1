// RoPE on bf16 rows (in place or into a copy) and per-row statistics for the exact score kernel (gfx950).
//
// Semantics of apply_rotary_emb (baseline/indexer.py:114-129) / the reference in-place RoPE kernel
// (optimized/indexer_project/op_kernel/fused_indexer_qk_reduce.asc:538-546,629-670): pairs (2j, 2j+1) of
// the rotated segment are complex-multiplied by (cos, sin) of the row's position in fp32 and rounded to
// bf16 (RNE).  Canonical order: y0 = fl(x0*c) - fl(x1*s), y1 = fl(x0*s) + fl(x1*c) (the library is built
// with -ffp-contract=off, so the products are rounded separately, exactly like the CPU oracle).
//
// Each lane owns 8 consecutive elements (one 16-byte load and store), so a row of D = 128 is 16 lanes and
// a wave covers 4 rows with fully coalesced accesses.  In stats mode the D/8 lanes of a row also reduce
// the row's squared norm and its smallest nonzero-element LSB exponent:
//   norm  >= ||row||_2 (rounded up),   span = ceil(log2 norm) - min_lsb_exponent.
// The score kernel uses norm for its MFMA error bound and span to prove that a double-precision
// recomputation of a dot product is exact.
#include "common.h"
#include "indexer_common.h"

namespace ks {
namespace {

__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float &y0, float &y1) {
  y0 = x0 * c - x1 * s;
  y1 = x0 * s + x1 * c;
}

template <bool STATS>
__global__ __launch_bounds__(256) void rope_rows_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst,
                                                       const float *__restrict__ freqs, int64_t rows, int D, int H,
                                                       int64_t S, int64_t pos0, int rope_start, int rope_dim,
                                                       float *__restrict__ norm, int32_t *__restrict__ span) {
  const int chunks_per_row = D / 8;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = c / chunks_per_row;
  const int j = static_cast<int>(c % chunks_per_row);
  const bool live = row < rows;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (live) v = *reinterpret_cast<const uint4 *>(src + row * D + 8 * j);
  const int e0 = 8 * j;
  if (live && rope_dim > 0 && e0 >= rope_start && e0 < rope_start + rope_dim) {
    const int64_t s = (row / H) % S;
    const float2 *cs = reinterpret_cast<const float2 *>(freqs) + (pos0 + s) * (rope_dim / 2) + (e0 - rope_start) / 2;
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float x0 = bf16_to_f32(static_cast<uint16_t>(w[p] & 0xFFFFu));
      const float x1 = bf16_to_f32(static_cast<uint16_t>(w[p] >> 16));
      const float2 t = cs[p];
      float y0, y1;
      rope_pair(x0, x1, t.x, t.y, y0, y1);
      w[p] = static_cast<uint32_t>(f32_to_bf16_rne(y0)) | (static_cast<uint32_t>(f32_to_bf16_rne(y1)) << 16);
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (live && dst != nullptr) *reinterpret_cast<uint4 *>(dst + row * D + 8 * j) = v;
  if constexpr (STATS) {
    // D in {64, 128}: the D/8 lanes of a row are an aligned group of the wave.
    float ss = 0.f;
    int lsb = 1 << 20;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint16_t b = static_cast<uint16_t>(h ? (w[p] >> 16) : (w[p] & 0xFFFFu));
        const float f = bf16_to_f32(b);
        ss += f * f;  // each square is exact (8-bit significand)
        if ((b & 0x7FFFu) != 0) lsb = min(lsb, bf16_lsb_exponent(b));
      }
    }
    for (int m = 1; m < chunks_per_row; m <<= 1) {
      ss += __shfl_xor(ss, m, 64);
      lsb = min(lsb, __shfl_xor(lsb, m, 64));
    }
    if (live && j == 0) {
      // fp32 sum of <= 128 squares: relative error < 2^-16; sqrt adds < 1 ulp; pad by 2^-12.
      const float nrm = ss > 0.f ? sqrtf(ss) * (1.0f + 0x1p-12f) : 0.f;
      norm[row] = nrm;
      int top = 0;
      if (nrm > 0.f) frexpf(nrm, &top);  // nrm < 2^top
      span[row] = nrm > 0.f ? top - lsb : 0;
    }
  }
}

}  // namespace

int launch_rope_rows(const uint16_t *src, uint16_t *dst, const float *freqs, int64_t rows, int D, int H, int64_t S,
                     int64_t pos0, int rope_start, int rope_dim, float *norm, int32_t *span, hipStream_t stream) {
  const int64_t chunks = rows * (D / 8);
  if (chunks == 0) return KS_OK;
  const int64_t blocks = ceil_div(chunks, 256);
  if (norm != nullptr) {
    hipLaunchKernelGGL(rope_rows_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, src, dst,
                       freqs, rows, D, H, S, pos0, rope_start, rope_dim, norm, span);
  } else {
    hipLaunchKernelGGL(rope_rows_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, src, dst,
                       freqs, rows, D, H, S, pos0, rope_start, rope_dim, norm, span);
  }
  KS_CHECK_LAUNCH("rope_rows_kernel");
  return KS_OK;
}

}  // namespace ks

extern "C" int ks_rope_inplace(uint16_t *x, const float *freqs, int64_t B, int64_t S, int64_t H, int64_t D,
                               int64_t rope_start, int64_t rope_dim, int64_t pos0, int64_t freq_rows, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && D >= 8, "ks_rope_inplace: bad shape B=%lld S=%lld H=%lld D=%lld",
               (long long)B, (long long)S, (long long)H, (long long)D);
  KS_CHECK_ARG(D % 8 == 0 && D <= 65536, "ks_rope_inplace: D=%lld must be a multiple of 8", (long long)D);
  KS_CHECK_ARG(rope_dim >= 0 && rope_dim % 8 == 0 && rope_start >= 0 && rope_start % 8 == 0 &&
                   rope_start + rope_dim <= D,
               "ks_rope_inplace: rotated segment [%lld, %lld) must be 8-aligned and inside [0, D)",
               (long long)rope_start, (long long)(rope_start + rope_dim));
  KS_CHECK_ARG(pos0 >= 0 && pos0 + S <= freq_rows, "ks_rope_inplace: positions [%lld, %lld) exceed freqs rows %lld",
               (long long)pos0, (long long)(pos0 + S), (long long)freq_rows);
  const int64_t rows = B * S * H;
  if (rows == 0 || rope_dim == 0) return KS_OK;
  KS_CHECK_ARG(x != nullptr && freqs != nullptr, "ks_rope_inplace: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16) && ks::aligned(freqs, 8), "ks_rope_inplace: x must be 16-byte aligned");
  return ks::launch_rope_rows(x, x, freqs, rows, static_cast<int>(D), static_cast<int>(H), S, pos0,
                              static_cast<int>(rope_start), static_cast<int>(rope_dim), nullptr, nullptr,
                              static_cast<hipStream_t>(stream));
}

extern "C" int ks_indexer_row_stats(const uint16_t *x, int64_t rows, int64_t D, float *norm, int32_t *span,
                                    void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(D == 128 || D == 64, "ks_indexer_row_stats: D=%lld, supported: 64 and 128", (long long)D);
  KS_CHECK_ARG(rows >= 0, "ks_indexer_row_stats: rows < 0");
  if (rows == 0) return KS_OK;
  KS_CHECK_ARG(x && norm && span, "ks_indexer_row_stats: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16), "ks_indexer_row_stats: x must be 16-byte aligned");
  return ks::launch_rope_rows(x, nullptr, nullptr, rows, static_cast<int>(D), 1, 1, 0, 0, 0, norm, span,
                              static_cast<hipStream_t>(stream));
}
