// Indexer score kernel (gfx950): bf16 MFMA q.k^T, exact bf16 rounding of every dot, ReLU, head-weighted
// reduction in the canonical order, causal mask.
//
// Semantics: baseline/indexer.py:176-193 (einsum -> relu_ -> * weights -> sum over heads -> -inf mask),
// replacing the reference megakernel optimized/indexer_project/op_kernel/fused_indexer_qk_reduce.asc:1-24,
// 368-428 (cube GEMM + vector head reduction).  Bit-exact contract (include/kswift.h): each dot is the
// exact real dot product rounded once to bf16; heads are summed in four groups g = (h/4) % 4, each in
// increasing h with fma (fp32 weights), then (G0 + G1) + (G2 + G3).
//
// Work decomposition: a 256-lane workgroup = 4 waves = 4 queries x one block of 256 keys.  The key block
// (64 KiB bf16) is staged once in LDS with a 16-byte XOR swizzle (chunk c of key r at c ^ (r & 15)), so the
// 16 lanes that read the same d-chunk of 16 different keys hit 16 distinct bank groups.  Each wave keeps its
// query's q rows (H heads x 128 d) as MFMA A-fragments in VGPRs and walks the block in 16-key tiles with
// v_mfma_f32_16x16x32_bf16 (M = 16 heads, N = 16 keys, 4 k-steps).  In the 16x16 output layout lane l holds
// heads 16m + 4(l/16) + r (r = 0..3) of key l % 16, i.e. exactly the canonical head group g = l/16, so the
// head sum runs in-lane and two xor-shuffles (16, 32) finish ((G0+G1)+(G2+G3)).
//
// Exactness: the MFMA fp32 sum A differs from the exact dot by less than
//   delta = C * 2^-23 * ||q_h|| * ||k_t||       (C = kScoreBoundC, measured error model),
// so RNE_bf16(A) is the exact answer unless a bf16 rounding boundary lies within delta of A.  Such "risky"
// dots (and every dot whose bf16 ulp is not >> delta) are recomputed exactly: 16 lanes form the 128 exact
// products in double precision and reduce them; the per-row spans from the statistics pass prove that every
// partial sum is representable (span_q + span_k <= 52), or a hi/lo split keeps both halves exact (<= 84).
#include "common.h"
#include "indexer_common.h"

namespace ks {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKB = 256;  // keys per workgroup block
constexpr int kWaves = 4; // queries per workgroup (one per wave)
constexpr int kD = 128;

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ float round_bf16_f(float a) { return bf16_to_f32(f32_to_bf16_rne(a)); }

// RNE to bf16 of the exact value a + b (two doubles).  TwoSum gives s + t == a + b exactly with
// s = fl(a + b); the bf16 grid is far coarser than the double grid, so RNE(a + b) = RNE(s) except when s
// is exactly a bf16 midpoint, where the sign of t decides (t == 0: ties to even).
__device__ uint16_t round2_to_bf16(double a, double b) {
  const double s = a + b;
  const double bb = s - a;
  const double t = (a - (s - bb)) + (b - bb);
  if (s == 0.0) return 0;
  const uint64_t bits = __builtin_bit_cast(uint64_t, s);
  const uint16_t sign = (bits >> 63) ? 0x8000 : 0;
  const uint64_t mag = bits & 0x7FFFFFFFFFFFFFFFull;
  const int e = static_cast<int>(mag >> 52) - 1023;
  const int tdir = (t == 0.0) ? 0 : (((t > 0.0) == (s > 0.0)) ? 1 : -1);  // residual, in magnitude
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

// Exact dot of one q row (global) and one key row (LDS, swizzled) by the 16 lanes of a group; lane j
// forms the products of elements 8j..8j+7.  Returns RNE_bf16(exact) as fp32 in every lane of the group.
__device__ float exact_dot16(const uint16_t *__restrict__ qrow, const uint4 *kl, int key_local, int j, int span_sum,
                             int top_sum, bool &ok) {
  const uint4 qa = *reinterpret_cast<const uint4 *>(qrow + 8 * j);
  const uint4 kb = kl[key_local * 16 + (j ^ (key_local & 15))];
  const uint32_t qw[4] = {qa.x, qa.y, qa.z, qa.w};
  const uint32_t kw[4] = {kb.x, kb.y, kb.z, kb.w};
  const bool split = span_sum > 52;
  const double thr = split ? ldexp(1.0, top_sum - 38) : 0.0;
  double hi = 0.0, lo = 0.0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const double a = bf16_to_f32(static_cast<uint16_t>(hh ? (qw[p] >> 16) : (qw[p] & 0xFFFFu)));
      const double b = bf16_to_f32(static_cast<uint16_t>(hh ? (kw[p] >> 16) : (kw[p] & 0xFFFFu)));
      const double prod = a * b;  // exact: 16 significant bits
      if (!split || fabs(prod) >= thr) hi += prod; else lo += prod;
    }
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    hi += __shfl_xor(hi, m, 64);
    lo += __shfl_xor(lo, m, 64);
  }
  ok = span_sum <= 84;
  return bf16_to_f32(round2_to_bf16(hi, lo));
}

template <int HT, bool WBF>
__global__ __launch_bounds__(256, 2) void indexer_scores_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const void *__restrict__ w,
    const float *__restrict__ qn, const int32_t *__restrict__ qsp, const float *__restrict__ kn,
    const int32_t *__restrict__ ksp, float *__restrict__ scores, int64_t S, int T, int64_t kbs, int causal,
    int64_t start_pos, int ratio, float bound_c, uint32_t *__restrict__ stats) {
  constexpr int H = HT * 16;
  __shared__ uint4 kl[kKB * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.z;
  const int kb0 = blockIdx.x * kKB;
  const int64_t s = static_cast<int64_t>(blockIdx.y) * kWaves + wave;
  const int nk = min(kKB, T - kb0);
  const int64_t krow0 = b * kbs + kb0;  // first key row of this block (also the stats row)

  // ---- stage the key block in LDS (zero rows past T)
  const uint16_t *kbase = k + krow0 * kD;
#pragma unroll 4
  for (int it = 0; it < kKB * 16 / 256; ++it) {
    const int lin = it * 256 + tid;
    const int kr = lin >> 4, ch = lin & 15;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (kr < nk) v = *reinterpret_cast<const uint4 *>(kbase + static_cast<int64_t>(kr) * kD + ch * 8);
    kl[kr * 16 + (ch ^ (kr & 15))] = v;
  }
  __syncthreads();
  if (s >= S) return;  // no barrier follows

  const int64_t limit = causal ? (start_pos + s + 1) / ratio : INT64_MAX;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t qrow0 = (b * S + s) * H;

  uint4 qa[HT][4];
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qa[m][kk] = *reinterpret_cast<const uint4 *>(q + (qrow0 + 16 * m + l16) * kD + 32 * kk + 8 * g);
  float wv[HT][4], dq[HT][4];
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t hrow = qrow0 + 16 * m + 4 * g + r;
      wv[m][r] = WBF ? bf16_to_f32(static_cast<const uint16_t *>(w)[hrow]) : static_cast<const float *>(w)[hrow];
      dq[m][r] = bound_c * 0x1p-23f * qn[hrow];
    }
  float *orow = scores + (b * S + s) * T;

  for (int n = 0; n < kKB / 16; ++n) {
    if (16 * n >= nk) break;
    const int key_local = 16 * n + l16;
    const int key = kb0 + key_local;
    const bool kvalid = key < T;
    if (kb0 + 16 * n >= limit) {  // whole tile masked (wave-uniform)
      if (g == 0 && kvalid) orow[key] = -INFINITY;
      continue;
    }
    f32x4_t acc[HT];
#pragma unroll
    for (int m = 0; m < HT; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint4 bv = kl[key_local * 16 + ((4 * kk + g) ^ l16)];
#pragma unroll
      for (int m = 0; m < HT; ++m) acc[m] = mfma16(qa[m][kk], bv, acc[m]);
    }
    const float knv = kvalid ? kn[krow0 + key_local] : 0.f;

    float dv[HT * 4];
    uint32_t risky = 0;
#pragma unroll
    for (int m = 0; m < HT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float A = acc[m][r];
        const float dl = dq[m][r] * knv;
        const float mid = __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, A) & 0xFFFF0000u) | 0x8000u);
        const bool rk = (A > -dl) && (fabsf(A - mid) < dl || fabsf(A) < 1024.f * dl);
        risky |= rk ? (1u << (4 * m + r)) : 0u;
        dv[4 * m + r] = round_bf16_f(A);
      }

    if (__ballot(risky != 0) != 0ull) {
#pragma unroll
      for (int i = 0; i < HT * 4; ++i) {
        uint64_t lm = __ballot((risky >> i) & 1u);
        while (lm != 0ull) {
          // up to four risky lanes per pass, one per 16-lane group
          uint64_t tmp = lm, batch = 0;
          int sel[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            sel[q4] = tmp ? __builtin_ctzll(tmp) : -1;
            if (tmp) {
              batch |= 1ull << sel[q4];
              tmp &= tmp - 1;
            }
          }
          lm = tmp;
          int L = g == 0 ? sel[0] : g == 1 ? sel[1] : g == 2 ? sel[2] : sel[3];
          if (L < 0) L = sel[0];  // idle groups repeat group 0's dot (result discarded)
          const int Lg = L >> 4, Ll = L & 15;
          const int m = i / 4, r = i % 4;
          const int64_t hrow = qrow0 + 16 * m + 4 * Lg + r;
          const int kls = 16 * n + Ll;
          int topq = 0, topk = 0;
          frexpf(qn[hrow], &topq);
          frexpf(kn[krow0 + kls], &topk);
          bool ok = true;
          const float ex = exact_dot16(q + hrow * kD, kl, kls, l16, qsp[hrow] + ksp[krow0 + kls], topq + topk, ok);
          const int rank = __builtin_popcountll(batch & ((1ull << lane) - 1ull));
          const float got = __shfl(ex, 16 * (rank < 4 ? rank : 3), 64);
          const bool okg = __shfl(ok ? 1 : 0, 16 * (rank < 4 ? rank : 3), 64) != 0;
          if ((batch >> lane) & 1ull) {
            if (okg) dv[i] = got;
          }
          if (stats != nullptr && lane == 0) {
            atomicAdd(&stats[0], static_cast<uint32_t>(__builtin_popcountll(batch)));
          }
          if (stats != nullptr && ((batch >> lane) & 1ull) && !okg) atomicAdd(&stats[1], 1u);
        }
      }
    }

    // ---- canonical head sum for this lane's group, then ((G0+G1)+(G2+G3))
    float G = 0.f;
#pragma unroll
    for (int m = 0; m < HT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float rv = fmaxf(dv[4 * m + r], 0.f);
        if constexpr (WBF) {
          G = G + round_bf16_f(rv * wv[m][r]);
        } else {
          G = __builtin_fmaf(rv, wv[m][r], G);
        }
      }
    const float s01 = G + __shfl_xor(G, 16, 64);
    float tot = s01 + __shfl_xor(s01, 32, 64);
    if constexpr (WBF) tot = round_bf16_f(tot);
    if (g == 0 && kvalid) orow[key] = (key < limit) ? tot : -INFINITY;
  }
}

template <int HT>
int launch_scores_ht(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                     const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B, int64_t S,
                     int64_t T, int64_t kbs, int causal, int64_t start_pos, int ratio, float bound_c, uint32_t *stats,
                     hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(ceil_div(T, kKB)), static_cast<unsigned>(ceil_div(S, kWaves)),
            static_cast<unsigned>(B));
  if (w_bf16) {
    hipLaunchKernelGGL((indexer_scores_kernel<HT, true>), grid, dim3(256), 0, stream, q, k, w, qn, qsp, kn, ksp,
                       scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c, stats);
  } else {
    hipLaunchKernelGGL((indexer_scores_kernel<HT, false>), grid, dim3(256), 0, stream, q, k, w, qn, qsp, kn, ksp,
                       scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c, stats);
  }
  KS_CHECK_LAUNCH("indexer_scores_kernel");
  return KS_OK;
}

}  // namespace

int launch_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                          const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B,
                          int64_t S, int64_t H, int64_t T, int64_t kbs, int causal, int64_t start_pos, int ratio,
                          float bound_c, uint32_t *stats, hipStream_t stream) {
  switch (H) {
    case 16:
      return launch_scores_ht<1>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos, ratio,
                                 bound_c, stats, stream);
    case 32:
      return launch_scores_ht<2>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos, ratio,
                                 bound_c, stats, stream);
    case 64:
      return launch_scores_ht<4>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos, ratio,
                                 bound_c, stats, stream);
    default:
      return fail(KS_ERR_INVALID, "indexer scores: H=%lld, supported: 16, 32, 64", (long long)H);
  }
}

}  // namespace ks

namespace {
int check_scores_args(const uint16_t *q, const uint16_t *k, const void *w, const float *qn, const int32_t *qsp,
                      const float *kn, const int32_t *ksp, float *scores, int64_t B, int64_t S, int64_t H, int64_t D,
                      int64_t T, int64_t kbs, int32_t ratio, int64_t start_pos) {
  KS_CHECK_ARG(D == 128, "ks_indexer_scores: D=%lld, the kernel is built for head_dim 128", (long long)D);
  KS_CHECK_ARG(H == 16 || H == 32 || H == 64, "ks_indexer_scores: H=%lld must be 16, 32 or 64", (long long)H);
  KS_CHECK_ARG(B >= 0 && S >= 0, "ks_indexer_scores: negative B or S");
  KS_CHECK_ARG(T >= 1 && T < (int64_t(1) << 31), "ks_indexer_scores: T=%lld out of range", (long long)T);
  KS_CHECK_ARG(kbs >= T, "ks_indexer_scores: k_batch_stride=%lld < T=%lld", (long long)kbs, (long long)T);
  KS_CHECK_ARG(ratio >= 1 && start_pos >= 0, "ks_indexer_scores: ratio must be >= 1 and start_pos >= 0");
  KS_CHECK_ARG(q && k && w && qn && qsp && kn && ksp && scores, "ks_indexer_scores: null pointer");
  KS_CHECK_ARG(ks::aligned(q, 16) && ks::aligned(k, 16) && ks::aligned(scores, 4),
               "ks_indexer_scores: q and k must be 16-byte aligned");
  return KS_OK;
}
}  // namespace

extern "C" int ks_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16,
                                 const float *q_norm, const int32_t *q_span, const float *k_norm,
                                 const int32_t *k_span, float *scores, int64_t B, int64_t S, int64_t H, int64_t D,
                                 int64_t T, int64_t k_batch_stride, int32_t causal, int64_t start_pos, int32_t ratio,
                                 void *stream) {
  ks::last_error().clear();
  int rc = check_scores_args(q, k, w, q_norm, q_span, k_norm, k_span, scores, B, S, H, D, T, k_batch_stride, ratio,
                             start_pos);
  if (rc != KS_OK) return rc;
  if (B * S == 0) return KS_OK;
  return ks::launch_indexer_scores(q, k, w, w_bf16 ? 1 : 0, q_norm, q_span, k_norm, k_span, scores, B, S, H, T,
                                   k_batch_stride, causal ? 1 : 0, start_pos, ratio, ks::kScoreBoundC, nullptr,
                                   static_cast<hipStream_t>(stream));
}

// Diagnostic variant (not part of the public header): explicit error-bound constant and a device counter
// pair stats[0] += exact recomputations, stats[1] += dots outside the provably exact range.
extern "C" int ks_dbg_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16,
                                     const float *q_norm, const int32_t *q_span, const float *k_norm,
                                     const int32_t *k_span, float *scores, int64_t B, int64_t S, int64_t H, int64_t D,
                                     int64_t T, int64_t k_batch_stride, int32_t causal, int64_t start_pos,
                                     int32_t ratio, float bound_c, uint32_t *stats, void *stream) {
  ks::last_error().clear();
  int rc = check_scores_args(q, k, w, q_norm, q_span, k_norm, k_span, scores, B, S, H, D, T, k_batch_stride, ratio,
                             start_pos);
  if (rc != KS_OK) return rc;
  if (B * S == 0) return KS_OK;
  return ks::launch_indexer_scores(q, k, w, w_bf16 ? 1 : 0, q_norm, q_span, k_norm, k_span, scores, B, S, H, T,
                                   k_batch_stride, causal ? 1 : 0, start_pos, ratio, bound_c, stats,
                                   static_cast<hipStream_t>(stream));
}
