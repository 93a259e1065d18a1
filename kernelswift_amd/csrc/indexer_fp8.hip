// FP8 (e4m3fn) rows for the indexer (gfx950): block quantisation of bf16 rows, and the dequantisation +
// row-statistics pass that feeds quantised q / k into the exact indexer.
//
// The reference configures its DeepSeek-style model with dtype = "fp8", scale_fmt = "ue8m0"
// (baseline/indexer.py:14-17): indexer q and k are stored as e4m3 codes with one fp32 scale per block of
// elements, the scale a power of two under ue8m0.  Quantisation (per block of `block` elements):
//   amax = max(max |x|, 1e-4);  s = amax * fp32(1/448)            (fp32 multiply, nearest even)
//   ue8m0: s = 2^ceil(log2 s)   (exponent of s, plus one when any mantissa bit is set)
//   code = e4m3_rne(clamp(x / s, -448, 448))                        (x / s: IEEE division, nearest even)
// and the value a code stands for is bf16(fp32(decode(code) * s)): exactly code * s when s is a power of
// two (e4m3 significands have 4 bits), so a ue8m0-quantised row dequantises without rounding.
//
// The indexer on quantised inputs is the bf16 indexer on those dequantised rows: the score kernels and the
// exact top-k are shared, and only this pass differs from the RoPE / statistics pass (quantised rows are
// stored after RoPE).  On the bounded path (64 heads, D = 128, fp32 weights) the score and recomputation
// kernels read the key codes themselves and this pass only forms the keys' statistics (q is dequantised here, once:
// the score kernel reads each query's rows from every key block's workgroup); elsewhere it writes the dequantised
// bf16 rows of both for the exact kernels.  The FP8 matrix instruction (v_mfma_scale_f32_16x16x128_f8f6f4) is not used for the
// scores: it aligns the 16 products of each of its steps to about 13 bits below the step's largest product
// (2^8 + 2^-6 - 2^8 gives 0; pinned by the GPU tests of the FP8 instruction model), which bounds its dot
// error far above the half-unit of bf16 that the exact selection needs to resolve.
#include "common.h"
#include "indexer_common.h"

namespace ks {

// e4m3fn code of a finite float y with |y| <= 448, rounded to nearest even (ties to the even code).
// Normal codes: value 2^(e-7) (1 + m/8), e in [1, 15] (e = 15, m = 7 is NaN); subnormal: m 2^-9.
__device__ __forceinline__ uint32_t e4m3_rne(float y) {
  const uint32_t u = __float_as_uint(y);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = __uint_as_float(u & 0x7FFFFFFFu);
  const int e = static_cast<int>((u >> 23) & 0xFFu) - 127;  // 2^e <= a < 2^(e+1) for normal fp32 a
  if (e < -6) {  // below the smallest normal 2^-6: multiples of 2^-9; q = 8 is the code of 2^-6 itself
    return sign | static_cast<uint32_t>(rintf(a * 0x1p9f));
  }
  // a / 2^(e-3) in [8, 16) exactly (scaling by a power of two); q = 16 carries into the exponent field
  const float q = rintf(a * __uint_as_float(static_cast<uint32_t>(127 + 3 - e) << 23));
  return sign | (static_cast<uint32_t>((e + 7) << 3) + static_cast<uint32_t>(q) - 8u);
}

namespace {

constexpr float kInv448 = 1.0f / 448.0f;  // fp32(1/448), rounded once

// One lane per 8 elements; LPB = block / 8 consecutive lanes share a scale (an aligned lane group, since a
// row holds a whole number of blocks).  Lanes past the end take part in the exchanges with zeros.
template <int LPB>
__global__ __launch_bounds__(256) void fp8_quant_kernel(const uint16_t *__restrict__ x, uint8_t *__restrict__ codes,
                                                        float *__restrict__ scales, uint32_t chunks, int ue8m0) {
  const uint32_t c = blockIdx.x * 256u + threadIdx.x;
  const bool live = c < chunks;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (live) v = reinterpret_cast<const uint4 *>(x)[c];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float xv[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    xv[2 * p] = bf16_to_f32(static_cast<uint16_t>(w[p] & 0xFFFFu));
    xv[2 * p + 1] = bf16_to_f32(static_cast<uint16_t>(w[p] >> 16));
  }
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xv[e]));
#define KS_MAX_STEP(S)                                                                    \
  if constexpr (LPB > S) {                                                                \
    amax = fmaxf(amax, __builtin_bit_cast(float, lane_xor<S>(__builtin_bit_cast(uint32_t, amax)))); \
  }
  KS_MAX_STEP(1)
  KS_MAX_STEP(2)
  KS_MAX_STEP(4)
  KS_MAX_STEP(8)
#undef KS_MAX_STEP
  amax = fmaxf(amax, 1e-4f);
  float s = amax * kInv448;
  if (ue8m0) {
    const uint32_t su = __float_as_uint(s);
    const uint32_t ex = ((su >> 23) & 0xFFu) + ((su & 0x7FFFFFu) != 0u ? 1u : 0u);  // biased ceil(log2 s)
    s = __uint_as_float(ex << 23);
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float y = fminf(fmaxf(__fdiv_rn(xv[e], s), -448.f), 448.f);
    const uint32_t code = e4m3_rne(y);
    if (e < 4) {
      lo |= code << (8 * e);
    } else {
      hi |= code << (8 * (e - 4));
    }
  }
  if (live) {
    reinterpret_cast<uint2 *>(codes)[c] = make_uint2(lo, hi);
    if (c % LPB == 0) scales[c / LPB] = s;
  }
}

struct Fp8RowJobK {
  const uint8_t *src;
  const float *scale;
  uint16_t *dst;
  float *norm;
  int32_t *span;
  int64_t src_batch_rows;
  uint32_t rows;
  FastDiv rpb;
};

Fp8RowJobK kernel_job(const Fp8RowJob &j) {
  Fp8RowJobK k{};
  k.src = j.src;
  k.scale = j.scale;
  k.dst = j.dst;
  k.norm = j.norm;
  k.span = j.span;
  k.src_batch_rows = j.src_batch_rows;
  k.rows = static_cast<uint32_t>(j.rows);
  k.rpb = FastDiv(static_cast<uint32_t>(j.rows_per_batch));
  return k;
}

// One lane per 8 elements (8 code bytes in, 16 bf16 bytes out, or none when dst is null: statistics only, for
// the kernels that read the codes themselves); the CPR = D / 8 lanes of a row reduce its statistics.  Blocks [0, blocks0) take job 0, the rest job 1 (fields selected one by one, uniformly).  The
// grid's threads also clear zero16 16-byte words at zero (grid-strided).
template <int CPR>
__global__ __launch_bounds__(256) void fp8_rows_kernel(Fp8RowJobK j0, Fp8RowJobK j1, uint32_t blocks0,
                                                      uint4 *__restrict__ zero, uint32_t zero16) {
  constexpr int D = 8 * CPR;
  const bool second = blockIdx.x >= blocks0;
#define KS_PICK(f) (second ? j1.f : j0.f)
  const uint8_t *__restrict__ src = KS_PICK(src);
  const float *__restrict__ scale = KS_PICK(scale);
  uint16_t *__restrict__ dst = KS_PICK(dst);
  const uint32_t rows = KS_PICK(rows);
  const int64_t sbr = KS_PICK(src_batch_rows);
  const FastDiv rpb = KS_PICK(rpb);
#undef KS_PICK
  const uint32_t blk = second ? blockIdx.x - blocks0 : blockIdx.x;
  const uint32_t c = blk * 256u + threadIdx.x;  // < 2^31 (checked on the host)
  const uint32_t row = c / CPR, j = c % CPR;
  const bool live = row < rows;
  const uint32_t rb = live ? rpb.div(row) : 0, rr = live ? row - rb * rpb.d : 0;
  const int64_t srow = static_cast<int64_t>(rb) * sbr + rr;
  uint2 raw = make_uint2(0, 0);
  float s = 0.f;
  if (live) {
    raw = *reinterpret_cast<const uint2 *>(src + srow * D + 8 * j);
    s = scale[srow];
  }
  // the hardware conversions (their exactness is pinned by the GPU tests): one instruction per two codes when every
  // scale of the wave is a power of two in range, else the exact value, an fp32 multiply and the RNE conversion
  const uint4 v = __builtin_amdgcn_ballot_w64(live && !fp8_scale_pow2(s)) == 0ull ? fp8_dequant8<true>(raw, s)
                                                                                  : fp8_dequant8<false>(raw, s);
  if (live && dst != nullptr) *reinterpret_cast<uint4 *>(dst + static_cast<int64_t>(row) * D + 8 * j) = v;
  float ss = 0.f;
  int lsb = 1 << 20;
  chunk_stats(v, ss, lsb);
  row_reduce<CPR>(ss, lsb);
  if (live && j == 0) {
    float *norm = second ? j1.norm : j0.norm;
    int32_t *span = second ? j1.span : j0.span;
    row_norm_span(ss, lsb, norm[row], span[row]);
  }
  // after the row's own stores, so that its loads do not wait behind these
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < zero16; i += gridDim.x * 256u) zero[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

int launch_fp8_rows(const Fp8RowJob &job0, const Fp8RowJob &job1, int D, hipStream_t stream, void *zero,
                    int64_t zero16) {
  KS_CHECK_ARG(D == 64 || D == 128, "fp8 rows: D=%d, supported: 64 and 128", D);
  KS_CHECK_ARG(zero16 >= 0 && zero16 < (int64_t(1) << 31) && (zero16 == 0 || aligned(zero, 16)),
               "fp8 rows: clear range of %lld words", (long long)zero16);
  const int64_t c0 = job0.rows * (D / 8), c1 = job1.rows * (D / 8);
  KS_CHECK_ARG(c0 + c1 + 512 < (int64_t(1) << 31), "fp8 rows: %lld + %lld chunks exceed the 32-bit grid",
               (long long)c0, (long long)c1);
  KS_CHECK_ARG(job0.rows_per_batch >= 1 && job1.rows_per_batch >= 1 && job0.rows_per_batch < (int64_t(1) << 31) &&
                   job1.rows_per_batch < (int64_t(1) << 31),
               "fp8 rows: rows per batch out of range");
  const int64_t b0 = ceil_div(c0, 256), b1 = ceil_div(c1, 256);
  KS_CHECK_ARG(b0 + b1 > 0 || zero16 == 0, "fp8 rows: a clear range needs rows");
  if (b0 + b1 == 0) return KS_OK;
  const dim3 grid(static_cast<unsigned>(b0 + b1));
  const Fp8RowJobK k0 = kernel_job(job0), k1 = kernel_job(job1);
  const uint32_t n0 = static_cast<uint32_t>(b0);
  uint4 *zp = static_cast<uint4 *>(zero);
  const uint32_t zn = static_cast<uint32_t>(zero16);
  if (D == 128) {
    hipLaunchKernelGGL(fp8_rows_kernel<16>, grid, dim3(256), 0, stream, k0, k1, n0, zp, zn);
  } else {
    hipLaunchKernelGGL(fp8_rows_kernel<8>, grid, dim3(256), 0, stream, k0, k1, n0, zp, zn);
  }
  KS_CHECK_LAUNCH("fp8_rows_kernel");
  return KS_OK;
}

}  // namespace ks

extern "C" int ks_fp8_quant_rows(const uint16_t *x, int64_t rows, int64_t D, int64_t block, int32_t ue8m0,
                                 uint8_t *codes, float *scales, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(block == 8 || block == 16 || block == 32 || block == 64 || block == 128,
               "ks_fp8_quant_rows: block=%lld, supported: 8, 16, 32, 64, 128", (long long)block);
  KS_CHECK_ARG(rows >= 0 && D >= block && D % block == 0,
               "ks_fp8_quant_rows: D=%lld must be a positive multiple of block=%lld", (long long)D, (long long)block);
  const int64_t chunks = rows * (D / 8);
  KS_CHECK_ARG(chunks + 256 < (int64_t(1) << 31), "ks_fp8_quant_rows: %lld rows of %lld exceed the 32-bit grid",
               (long long)rows, (long long)D);
  if (rows == 0) return KS_OK;
  KS_CHECK_ARG(x && codes && scales, "ks_fp8_quant_rows: null pointer");
  KS_CHECK_ARG(ks::aligned(x, 16) && ks::aligned(codes, 8) && ks::aligned(scales, 4),
               "ks_fp8_quant_rows: x must be 16-byte aligned, codes 8-byte aligned");
  const dim3 grid(static_cast<unsigned>(ks::ceil_div(chunks, 256)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint32_t n = static_cast<uint32_t>(chunks);
  const int u = ue8m0 ? 1 : 0;
  switch (block) {
    case 8: hipLaunchKernelGGL(ks::fp8_quant_kernel<1>, grid, dim3(256), 0, st, x, codes, scales, n, u); break;
    case 16: hipLaunchKernelGGL(ks::fp8_quant_kernel<2>, grid, dim3(256), 0, st, x, codes, scales, n, u); break;
    case 32: hipLaunchKernelGGL(ks::fp8_quant_kernel<4>, grid, dim3(256), 0, st, x, codes, scales, n, u); break;
    case 64: hipLaunchKernelGGL(ks::fp8_quant_kernel<8>, grid, dim3(256), 0, st, x, codes, scales, n, u); break;
    default: hipLaunchKernelGGL(ks::fp8_quant_kernel<16>, grid, dim3(256), 0, st, x, codes, scales, n, u); break;
  }
  KS_CHECK_LAUNCH("fp8_quant_kernel");
  return KS_OK;
}
