// RoPE on bf16 rows (in place or into a copy) and per-row statistics for the exact score kernel (gfx950).
//
// Semantics of apply_rotary_emb (baseline/indexer.py:114-129) / the reference in-place RoPE kernel
// (optimized/indexer_project/op_kernel/fused_indexer_qk_reduce.asc:538-546,629-670): pairs (2j, 2j+1) of
// the rotated segment are complex-multiplied by (cos, sin) of the row's position in fp32 and rounded to
// bf16 (RNE).  Canonical order: y0 = fl(x0*c) - fl(x1*s), y1 = fl(x0*s) + fl(x1*c) (the library is built
// with -ffp-contract=off, so the products are rounded separately, exactly like the CPU oracle).
//
// A lane owns 16-byte chunks of 8 consecutive elements: one in the generic form; two of one row in stats mode
// (chunks j and j + D/16 of the row's D/16 lanes, so a wave's loads and stores cover whole rows, coalesced).  In
// stats mode the lanes of a row also reduce the row's squared norm and its smallest nonzero-element LSB
// exponent:
//   norm  >= ||row||_2 (rounded up),   span = ceil(log2 norm) - min_lsb_exponent.
// The score kernel uses norm for its MFMA error bound and span to prove that a double-precision
// recomputation of a dot product is exact.
#include "common.h"
#include "indexer_common.h"

namespace ks {
namespace {

// Kernel-side form of a RowJob: 32-bit row arithmetic with precomputed divisors.
struct RowJobK {
  const uint16_t *src;
  uint16_t *dst;
  float *norm;
  int32_t *span;
  int64_t src_batch_rows, pos0;
  uint32_t rows;
  int rope_dim;
  int rotated_only;
  FastDiv rpb, H, S;
};

RowJobK kernel_job(const RowJob &j) {
  RowJobK k{};
  k.src = j.src;
  k.dst = j.dst;
  k.norm = j.norm;
  k.span = j.span;
  k.src_batch_rows = j.src_batch_rows;
  k.pos0 = j.pos0;
  k.rows = static_cast<uint32_t>(j.rows);
  k.rope_dim = j.rope_dim;
  k.rotated_only = j.rotated_only;
  k.rpb = FastDiv(static_cast<uint32_t>(j.rows_per_batch));
  k.H = FastDiv(static_cast<uint32_t>(j.H));
  k.S = FastDiv(static_cast<uint32_t>(j.S));
  return k;
}

// Threads own 16-byte chunks: one each in the generic form (CPR 0: any D, no statistics), two of the same row in
// the statistics forms (CPR = chunks per row, 8 or 16: lane j of the row's CPR / 2 lanes holds chunks j and
// j + CPR / 2), so that the row and position arithmetic, the statistics' final steps and the weight scaling are
// shared by twice the bytes.  Blocks [0, blocks0) take job 0 and the rest job 1 (a uniform choice, so each field is
// selected separately from the kernel arguments, never through a pointer to them).  The grid's threads also clear
// zero16 16-byte words at zero (grid-strided).
template <int CPR>
__global__ __launch_bounds__(256) void rope_rows_kernel(RowJobK j0, RowJobK j1, uint32_t blocks0,
                                                       const float *__restrict__ freqs, int D, FastDiv cpr,
                                                       int rope_start, uint4 *__restrict__ zero, uint32_t zero16,
                                                       WeightScale wsc) {
  constexpr int NC = CPR == 0 ? 1 : 2;  // chunks per thread
  constexpr int LPR = CPR / NC;         // lanes per row (statistics forms)
  const bool second = blockIdx.x >= blocks0;
#define KS_PICK(f) (second ? j1.f : j0.f)
  const uint16_t *__restrict__ src = KS_PICK(src);
  uint16_t *__restrict__ dst = KS_PICK(dst);
  const uint32_t rows = KS_PICK(rows);
  const int64_t sbr = KS_PICK(src_batch_rows);
  const int64_t pos0 = KS_PICK(pos0);
  const int rope_dim = KS_PICK(rope_dim);
  const bool rotated_only = KS_PICK(rotated_only) != 0;
  const FastDiv rpb = KS_PICK(rpb), Hd = KS_PICK(H), Sd = KS_PICK(S);
#undef KS_PICK
  const uint32_t blk = second ? blockIdx.x - blocks0 : blockIdx.x;
  const uint32_t c = blk * 256u + threadIdx.x;  // < 2^31 (checked on the host)
  uint32_t row, j;
  if constexpr (CPR == 0) {
    row = cpr.div(c);
    j = c - row * cpr.d;
  } else {
    row = c / LPR;  // powers of two: shifts
    j = c % LPR;
  }
  const bool live = row < rows;
  const uint32_t rb = live ? rpb.div(row) : 0, rr = live ? row - rb * rpb.d : 0;
  const int64_t srow = static_cast<int64_t>(rb) * sbr + rr;
  // both chunks' loads go out before any use
  uint4 v[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    v[i] = make_uint4(0, 0, 0, 0);
    if (live) v[i] = *reinterpret_cast<const uint4 *>(src + srow * D + 8 * (j + i * LPR));
  }
  bool any_rot = false;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e0 = 8 * static_cast<int>(j + i * LPR);
    any_rot = any_rot || (rope_dim > 0 && e0 >= rope_start && e0 < rope_start + rope_dim);
  }
  if (live && any_rot) {
    const uint32_t t = Hd.div(rr);
    const int64_t pos = pos0 + (t - Sd.div(t) * Sd.d);
    const float2 *cs0 = reinterpret_cast<const float2 *>(freqs) + pos * (rope_dim / 2);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e0 = 8 * static_cast<int>(j + i * LPR);
      if (e0 >= rope_start && e0 < rope_start + rope_dim) v[i] = rope_chunk(v[i], cs0 + (e0 - rope_start) / 2);
    }
  }
  if (live && dst != nullptr) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e0 = 8 * static_cast<int>(j + i * LPR);
      if (!rotated_only || (e0 >= rope_start && e0 < rope_start + rope_dim))
        *reinterpret_cast<uint4 *>(dst + static_cast<int64_t>(row) * D + e0) = v[i];
    }
  }
  if constexpr (CPR != 0) {
    // the LPR lanes of a row are an aligned group of the wave
    float ss = 0.f;
    uint32_t mmin = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < NC; ++i) chunk_stats_packed(v[i], ss, mmin);
    int lsb = lsb_of_min(mmin);
    row_reduce<LPR>(ss, lsb);
    if (live && j == 0) {
      float *norm = second ? j1.norm : j0.norm;
      int32_t *span = second ? j1.span : j0.span;
      row_norm_span(ss, lsb, norm[row], span[row]);
    }
  }
  // the first job's head weights scaled, one per row (torch's rounding of a tensor times a Python float)
  if (wsc.out != nullptr && !second && live && j == 0) {
    if (wsc.bf16) {
      const float x = bf16_to_f32(static_cast<const uint16_t *>(wsc.w)[row]) * wsc.scale;
      static_cast<uint16_t *>(wsc.out)[row] = f32_to_bf16_rne(x);
    } else {
      static_cast<float *>(wsc.out)[row] = static_cast<const float *>(wsc.w)[row] * wsc.scale;
    }
  }
  // after the row's own stores, so that its loads do not wait behind these
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < zero16; i += gridDim.x * 256u) zero[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

int launch_rope_rows(const RowJob &job0, const RowJob &job1, const float *freqs, int D, int rope_start,
                     hipStream_t stream, void *zero, int64_t zero16, const WeightScale *wscale) {
  KS_CHECK_ARG(zero16 >= 0 && zero16 < (int64_t(1) << 31) && (zero16 == 0 || aligned(zero, 16)),
               "rope rows: clear range of %lld words", (long long)zero16);
  const bool stats = job0.norm != nullptr;
  const int64_t tpr = stats ? D / 16 : D / 8;  // threads per row: two chunks each with statistics, else one
  const int64_t c0 = job0.rows * tpr, c1 = job1.rows * tpr;
  KS_CHECK_ARG(c0 + c1 + 512 < (int64_t(1) << 31), "rope rows: %lld + %lld chunks exceed the 32-bit grid",
               (long long)c0, (long long)c1);
  KS_CHECK_ARG(job0.rows_per_batch >= 1 && job1.rows_per_batch >= 1 && job0.H >= 1 && job1.H >= 1 &&
                   job0.S >= 1 && job1.S >= 1 && job0.rows_per_batch < (int64_t(1) << 31) &&
                   job1.rows_per_batch < (int64_t(1) << 31) && job0.H < (int64_t(1) << 31) &&
                   job1.H < (int64_t(1) << 31) && job0.S < (int64_t(1) << 31) && job1.S < (int64_t(1) << 31),
               "rope rows: batch, head or position extent out of range");
  const int64_t b0 = ceil_div(c0, 256), b1 = ceil_div(c1, 256);
  KS_CHECK_ARG(b0 + b1 > 0 || zero16 == 0, "rope rows: a clear range needs rows");
  if (b0 + b1 == 0) return KS_OK;
  KS_CHECK_ARG((job1.rows == 0 || (job1.norm != nullptr) == stats) && (!stats || D == 64 || D == 128),
               "rope rows: statistics need D in {64, 128} and both jobs alike");
  const dim3 grid(static_cast<unsigned>(b0 + b1));
  const RowJobK k0 = kernel_job(job0), k1 = kernel_job(job1);
  const FastDiv cpr(static_cast<uint32_t>(D / 8));
  const uint32_t n0 = static_cast<uint32_t>(b0);
  uint4 *zp = static_cast<uint4 *>(zero);
  const uint32_t zn = static_cast<uint32_t>(zero16);
  const WeightScale ws = wscale != nullptr ? *wscale : WeightScale{nullptr, nullptr, 1.f, 0};
  if (stats && D == 128) {
    hipLaunchKernelGGL(rope_rows_kernel<16>, grid, dim3(256), 0, stream, k0, k1, n0, freqs, D, cpr, rope_start, zp, zn, ws);
  } else if (stats) {
    hipLaunchKernelGGL(rope_rows_kernel<8>, grid, dim3(256), 0, stream, k0, k1, n0, freqs, D, cpr, rope_start, zp, zn, ws);
  } else {
    hipLaunchKernelGGL(rope_rows_kernel<0>, grid, dim3(256), 0, stream, k0, k1, n0, freqs, D, cpr, rope_start, zp, zn, ws);
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
  const ks::RowJob job{x, x, nullptr, nullptr, rows, rows, rows, H, S, pos0, static_cast<int>(rope_dim)};
  const ks::RowJob none{nullptr, nullptr, nullptr, nullptr, 0, 1, 0, 1, 1, 0, 0};
  return ks::launch_rope_rows(job, none, freqs, static_cast<int>(D), static_cast<int>(rope_start),
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
  const ks::RowJob job{x, nullptr, norm, span, rows, rows, rows, 1, 1, 0, 0};
  const ks::RowJob none{nullptr, nullptr, nullptr, nullptr, 0, 1, 0, 1, 1, 0, 0};
  return ks::launch_rope_rows(job, none, nullptr, static_cast<int>(D), 0, static_cast<hipStream_t>(stream));
}
