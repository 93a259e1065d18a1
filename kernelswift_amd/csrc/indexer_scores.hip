// Indexer score kernel (gfx950): bf16 MFMA q.k^T, exact bf16 rounding of every dot, ReLU, head-weighted
// reduction in the canonical order, causal mask.
//
// Semantics: baseline/indexer.py:176-193 (einsum -> relu_ -> * weights -> sum over heads -> -inf mask),
// replacing the reference megakernel optimized/indexer_project/op_kernel/fused_indexer_qk_reduce.asc:1-24,
// 368-428 (cube GEMM + vector head reduction).  Bit-exact contract (include/kswift.h): each dot is the
// exact real dot product rounded once to bf16; heads are summed in four groups g = (h/4) % 4, each in
// increasing h with fma (fp32 weights), then (G0 + G1) + (G2 + G3).
//
// Work decomposition: a 512-lane workgroup = 8 waves = 8 queries x a block of 256 keys.  The key block is
// staged once in LDS (64 KiB; rows past T unused) behind the kernel's only barrier; from there each wave runs
// independently.  A wave keeps its query's rows in VGPRs as MFMA A-fragments and walks the block in
// 16-key tiles with v_mfma_f32_16x16x32_bf16 (M = 16 heads, N = 16 keys, 4 k-steps), issuing the next
// tile's MFMAs before the current tile's epilogue.  LDS rows use a 16-byte XOR swizzle (chunk c of row r
// at c ^ (r & 15)), so 16 lanes reading one chunk of 16 rows hit 16 distinct bank groups.  In the MFMA
// output layout lane l holds heads 16m + 4(l/16) + r (r = 0..3) of key l % 16, i.e. exactly the canonical
// head group g = l/16, so the head sum runs in-lane and two permlane swaps finish ((G0+G1)+(G2+G3)).
//
// Exactness: the MFMA fp32 sum A differs from the exact dot by at most the half-width
//   delta = C * 2^-23 * (||q_h|| + 2^-122)(max_t ||k_t|| + 2^-122) + 2^-144   (C = score_bound_c(D): 13 for
//   D = 128, 9 for D = 64),
// derived from the instruction's accumulation (see dot_halfwidth), so the relu'd bf16 value is exact when
// RNE(A - delta) and RNE(A + delta) agree after the ReLU (one packed convert and one packed max per pair of
// dots and interval end).  Keys with a disagreeing ("near-tie") dot are deferred: both interval ends of all
// their head groups go to a per-wave LDS list, and when the list fills (and at the end) the near-tie dots
// are recomputed exactly, 16 at a time with 4 lanes per dot, and the affected scores rewritten.  Per-row
// spans from the statistics pass prove every partial sum of the exact dot representable in a double
// (span_q + span_k <= 52); up to 84 a hi/lo split keeps both halves exact; beyond that an integer
// accumulator (exact_dot_wide_bf16) computes the dot.  A wave whose norms could overflow inside the MFMA
// ((||q|| ||k|| >= 2^126) treats every dot as a near tie.
//
// Bound mode (BOUND) keeps the interval test but writes, instead of recomputing near ties, the canonical score
// of the lower interval ends and a bound U on its distance from the exact score; its counting form (COUNT) also
// builds each row's histogram of the first 11-bit digit of the lower ends' keys for the bounded top-k's
// threshold (per-wave LDS counts, flushed with one global atomic per nonzero bucket).
//
// FP8 keys (F8, bound mode): k holds e4m3 codes with one fp32 scale per row, read directly (half the bytes of
// bf16 rows) and dequantised in registers to the bf16 rows the contract defines, bf16(fp32(value * scale)), before
// the key block is staged in LDS; the rest of the kernel is the bf16 one.  (q arrives dequantised: each query's
// rows are read by every key block's workgroup, T / 256 of them, so they are converted once, by the statistics
// pass, while a key block is read by S / 8 workgroups.)
#include "common.h"
#include "indexer_common.h"
#include "indexer_exact.h"

#include <type_traits>

namespace ks {
namespace {


constexpr int kQW = 8;        // queries (= waves) per workgroup
constexpr int kThreads = kQW * 64;
constexpr int kKR = kScoreKeyBlock;  // keys per workgroup
constexpr int kEntCap = 32;   // deferred key entries per wave (flushed before another 16 could overflow them)
static_assert(kEntCap >= 16, "16 listed keys are resolved at a time");
static_assert(4 * kEntCap <= 255, "list entries hold the (entry, group) pair in 8 bits");
constexpr int kDotCap = 256;  // near-tie dots listed at a time per wave

// Context of one key whose score depends on a near-tie dot: for the four head groups, the relu'd bf16
// values of the two interval ends (packed pairs, 2 HT per group; they differ exactly at the near-tie slots).
// Sized by the head count, so that fewer heads leave LDS for a second workgroup per CU.
template <int HT>
struct alignas(16) KeyEntry {
  uint32_t pl[4][2 * HT];
  uint32_t ph[4][2 * HT];
  int32_t key;
  int32_t pad[3];
};

template <int KD, int HT>
struct ScoresLds {
  uint4 k[kKR * KD / 8];             // swizzled key block of this workgroup (KD / 8 16-byte chunks per key)
  uint16_t kstep[HT == 1 ? kKR : 0][KD / 8];  // 16 heads: per key, the step exponents of |k| (step_exponent_pow2 of
                                              // each 16-byte chunk: a chunk is one accumulation step)
  uint8_t klist[kQW][kKR];           // per wave: block rows of the keys holding a near-tie dot (a wave's tiles
                                     // defer at most every key of the block)
  KeyEntry<HT> ent[HT == 1 ? 0 : kQW][kEntCap];  // 16 heads: the resolution keeps its keys' values in registers
  uint32_t dots[kQW][kDotCap];       // near-tie dots: head << 24 | key row << 16 | pair << 4 | slot,
                                     // pair = 4 entry + group
  int32_t kspan[kKR];                // row statistics of the key block and of each wave's query rows, for
  float knorm[kKR];                  // the exact recomputation (no global loads there)
  int32_t qspan[kQW][64];
  float qnorm[kQW][64];
  float dl[kQW][64];                 // each wave's interval half-widths, one per head
  float w[kQW][64];                  // each wave's head weights (fp32)
};

// Canonical sum of one lane's head group (heads 16 m + 4 g + r, m = 0 .. HT - 1, r = 0 .. 3, in that order) from
// the relu'd bf16 values word(2 m + r / 2) (packed pairs): fp32 weights, G = fma(r_h, w_h, G); bf16 weights,
// G = G + bf16(r_h w_h), the two products of a pair rounded together by one v_cvt_pk_bf16_f32 (RNE, the same
// results as the software rounding for every non-NaN value) and added in head order.
template <int HT, bool WBF, typename Word>
__device__ __forceinline__ float group_sum(Word word, const float (&wv)[HT][4]) {
  float G = 0.f;
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int rp = 0; rp < 2; ++rp) {
      const uint32_t p2 = word(2 * m + rp);
      if constexpr (WBF) {
        const uint32_t pr = cvt_pk_bf16(unpack_lo(p2) * wv[m][2 * rp], unpack_hi(p2) * wv[m][2 * rp + 1]);
        G = G + unpack_lo(pr);
        G = G + unpack_hi(pr);
      } else {
        G = __builtin_fmaf(unpack_lo(p2), wv[m][2 * rp], G);
        G = __builtin_fmaf(unpack_hi(p2), wv[m][2 * rp + 1], G);
      }
    }
  return G;
}

// Exclusive prefix sum over the 64 lanes of a wave of values below 2^NB, and the wave's total: one ballot per bit
// and the count of the lanes below (mbcnt), with no data moved between lanes.
template <int NB>
__device__ __forceinline__ uint32_t wave_excl_scan_bits(uint32_t v, uint32_t &total) {
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint64_t m = __builtin_amdgcn_ballot_w64((v >> b) & 1u);
    pre += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u))
           << b;
    tot += static_cast<uint32_t>(__builtin_popcountll(m)) << b;
  }
  total = tot;
  return pre;
}

// A score's bf16 rounding (bf16 weights) with the hardware conversion: RNE, the same as the software rounding for
// every non-NaN value.
__device__ __forceinline__ float round_score_bf16(float x) { return unpack_lo(cvt_pk_bf16(x, x)); }

// Near-tie slot bits (16 per head group) of an entry: positions where the two interval ends differ.
template <int HT>
__device__ __forceinline__ uint32_t entry_mask(const KeyEntry<HT> &en, int gg) {
  uint32_t m = 0;
#pragma unroll
  for (int p = 0; p < 2 * HT; ++p) {
    const uint32_t x = en.pl[gg][p] ^ en.ph[gg][p];
    m |= ((x & 0xFFFFu) ? 1u : 0u) << (2 * p);
    m |= ((x >> 16) ? 1u : 0u) << (2 * p + 1);
  }
  return m;
}

// The exact value (RNE to bf16, before the ReLU) of the dot of head h's q row and key row kl of the block,
// computed by a quad of lanes (this lane: quarter `sub`); every lane of the wave calls it together (the path
// choices are ballots).  16 heads: quarter `sub` takes the 16-byte chunks 4c + sub, which lane h + 16 sub holds as
// its A-fragment qa[0][c] (read with ds_bpermute); more heads: the chunks kLC sub + c, read from global memory
// (L2-resident).  scur: the span sum that decided the path (> 84: the integer accumulator).
template <int HT, int KD>
__device__ __forceinline__ uint16_t quad_exact_dot(ScoresLds<KD, HT> &L, int wave, int sub, int h, int kl,
                                                   const uint16_t *__restrict__ q, QSplit qsp,
                                                   const uint4 (&qa)[HT][KD / 32], int64_t qrow0, int &scur) {
  constexpr int kC = KD / 8, kLC = KD / 32;  // 16-byte chunks per key row; chunks per lane
  // the q rows this lane reads from memory: its quarter (elements KD/4 sub ..) lies wholly on one side of a
  // split (QSplit boundaries are 32-aligned)
  const uint16_t *qsrc = (qsp.rot != nullptr && (KD / 4) * sub >= qsp.lo && (KD / 4) * sub < qsp.hi) ? qsp.rot : q;
  uint4 qcur[kLC], kcur[kLC];
  if constexpr (HT == 1) {
    const int src = 4 * (h + 16 * sub);
    auto bp = [&](uint32_t v) { return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(v))); };
#pragma unroll
    for (int c = 0; c < kLC; ++c) {
      qcur[c] = make_uint4(bp(qa[0][c].x), bp(qa[0][c].y), bp(qa[0][c].z), bp(qa[0][c].w));
      kcur[c] = L.k[kl * kC + ((4 * c + sub) ^ (kl & (kC - 1)))];
    }
  } else {
    const uint4 *qp = reinterpret_cast<const uint4 *>(qsrc + (qrow0 + h) * KD + (KD / 4) * sub);
#pragma unroll
    for (int c = 0; c < kLC; ++c) qcur[c] = qp[c];
#pragma unroll
    for (int c = 0; c < kLC; ++c) kcur[c] = L.k[kl * kC + ((kLC * sub + c) ^ (kl & (kC - 1)))];
  }
  scur = L.qspan[wave][h] + L.kspan[kl];
  uint16_t r;
  if (__builtin_amdgcn_ballot_w64(scur > 52) == 0ull) {
    // every partial sum is a multiple of the smallest product LSB and below 2^53 of it: exact doubles
    // in any order
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int c = 0; c < kLC; ++c) {
      const uint32_t qw[4] = {qcur[c].x, qcur[c].y, qcur[c].z, qcur[c].w};
      const uint32_t kw[4] = {kcur[c].x, kcur[c].y, kcur[c].z, kcur[c].w};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        a0 = __builtin_fma(static_cast<double>(unpack_lo(qw[p])), static_cast<double>(unpack_lo(kw[p])), a0);
        a1 = __builtin_fma(static_cast<double>(unpack_hi(qw[p])), static_cast<double>(unpack_hi(kw[p])), a1);
      }
    }
    const double sum = quad_sum_f64(a0 + a1);
    const bool outside = sum != 0.0 && !(fabs(sum) >= 0x1p-126 && fabs(sum) < 0x1p127);
    if (__builtin_amdgcn_ballot_w64(outside) == 0ull) {
      r = round_to_bf16_fast(sum);
    } else {
      r = round_dir_to_bf16(sum, 0);
    }
  } else {
    // wide dynamic range: products above / below 2^(top - 38) accumulate separately, each exactly
    const int span_sum = scur;
    const int top_sum = frexp_exp(L.qnorm[wave][h]) + frexp_exp(L.knorm[kl]);
    const bool split = span_sum > 52;
    const double thr = split ? ldexp(1.0, top_sum - 38) : 0.0;
    double hi = 0.0, lo = 0.0;
    // rare path, kept register-light: one dword of q and k per step, re-read from memory
    const uint32_t *q32 = reinterpret_cast<const uint32_t *>(qsrc + (qrow0 + h) * KD + (KD / 4) * sub);
#pragma unroll 1
    for (int j = 0; j < 4 * kLC; ++j) {
      const uint32_t qw = q32[j];
      const uint32_t kw =
          reinterpret_cast<const uint32_t *>(&L.k[kl * kC + ((kLC * sub + (j >> 2)) ^ (kl & (kC - 1)))])[j & 3];
      const double p0 = static_cast<double>(unpack_lo(qw)) * static_cast<double>(unpack_lo(kw));
      const double p1 = static_cast<double>(unpack_hi(qw)) * static_cast<double>(unpack_hi(kw));
      if (!split || fabs(p0) >= thr) hi += p0; else lo += p0;
      if (!split || fabs(p1) >= thr) hi += p1; else lo += p1;
    }
    r = round2_to_bf16(quad_sum_f64(hi), quad_sum_f64(lo));
  }
  if (scur > 84) {
    // wider still (the whole quad takes this branch): the integer accumulator, any range
    const uint32_t *q32 = reinterpret_cast<const uint32_t *>(qsrc + (qrow0 + h) * KD);  // part `sub` of it
    r = exact_dot_wide_bf16<KD, 4>(
        [&](int j) { return q32[j]; },
        [&](int j) {
          return reinterpret_cast<const uint32_t *>(&L.k[kl * kC + ((j >> 2) ^ (kl & (kC - 1)))])[j & 3];
        },
        sub);
  }
  return r;
}

// Exact recomputation of the deferred near-tie dots of one wave, then of the affected scores.
template <int HT, int KD, bool WBF>
__device__ void flush_entries(ScoresLds<KD, HT> &L, int wave, int lane, int nent, const uint16_t *__restrict__ q,
                              const uint4 (&qa)[HT][KD / 32], int64_t qrow0, float *orow, int64_t limit, int T, int kb0,
                              const float (&wv)[HT][4], uint32_t &n_exact, uint32_t &n_unres, QSplit qsp) {
  KeyEntry<HT> *E = L.ent[wave];
  uint32_t *D = L.dots[wave];
  const int g = lane >> 4, l16 = lane & 15;
  // 1. near-tie masks of the (entry, group) pairs, pair = 4 * entry + group; taken before any patching
  const int npairs = 4 * nent;
  auto key_row = [&](int pair) {  // row of the entry's key in the LDS block (entries hold keys of the block)
    return static_cast<uint32_t>(min(max(E[pair >> 2].key - kb0, 0), kKR - 1));
  };
  // pairs are taken 64 at a time: pair 64 i + lane in set i
  constexpr int kSets = (4 * kEntCap + 63) / 64;
  uint32_t mset[kSets], rset[kSets], cset[kSets], first[kSets];
  uint32_t ndots_u = 0;
#pragma unroll
  for (int i = 0; i < kSets; ++i) {
    const int pair = 64 * i + lane;
    mset[i] = pair < npairs ? entry_mask<HT>(E[pair >> 2], pair & 3) : 0u;
    rset[i] = pair < npairs ? key_row(pair) : 0u;
    cset[i] = __builtin_popcount(mset[i]);  // at most 4 HT near-tie slots per pair
    uint32_t tot;
    first[i] = ndots_u + wave_excl_scan_bits<HT == 1 ? 3 : HT == 2 ? 4 : 5>(cset[i], tot);  // list position of the
    ndots_u += tot;                                                                       // pair's first dot
  }
  const int ndots = static_cast<int>(ndots_u);
  n_exact += ndots_u;
  // 2. the dot list, kDotCap at a time: exact dots, 16 per pass, 4 lanes per dot (lane quarter `sub` owns
  //    elements KD/4 sub .. KD/4 (sub + 1) - 1); the exact relu'd value replaces the pl value of its slot.
  //    List entry: head (slot s of pair (entry, group gg) is head 16 (s >> 2) + 4 gg + (s & 3)), key row,
  //    pair and slot, so that one LDS read locates both operands.
  constexpr int kC = KD / 8, kLC = KD / 32;  // 16-byte chunks per key row; chunks per lane
  auto pack = [](uint32_t pair, uint32_t row, int bit) {
    const uint32_t h = 16u * (bit >> 2) + 4u * (pair & 3u) + (bit & 3);
    return (h << 24) | (row << 16) | (pair << 4) | static_cast<uint32_t>(bit);
  };
  for (int base = 0; base < ndots; base += kDotCap) {
#pragma unroll
    for (int i = 0; i < kSets; ++i) {
      uint32_t mm = mset[i];
      int pos = static_cast<int>(first[i]) - base;
      while (mm) {
        const int bit = __builtin_ctz(mm);
        mm &= mm - 1;
        if (pos >= 0 && pos < kDotCap) D[pos] = pack(static_cast<uint32_t>(64 * i + lane), rset[i], bit);
        ++pos;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nd = min(kDotCap, ndots - base);
    const int dq = lane >> 2, sub = lane & 3;
    for (int b0 = 0; b0 < nd; b0 += 16) {
      // list entry of this quad (idle quads repeat the last one; the result is identical)
      const uint32_t dcur = D[min(b0 + dq, nd - 1)];
      const int h = static_cast<int>(dcur >> 24), kl = static_cast<int>((dcur >> 16) & 255u);
      const int pr = static_cast<int>((dcur >> 4) & 255u), slot = static_cast<int>(dcur & 15u);
      int scur;
      const uint16_t r = quad_exact_dot<HT, KD>(L, wave, sub, h, kl, q, qsp, qa, qrow0, scur);
      const uint32_t rv = (r & 0x8000) ? 0u : r;  // ReLU (also maps -0 to +0)
      if (sub == 0 && b0 + dq < nd) {
        uint16_t *half = reinterpret_cast<uint16_t *>(&E[pr >> 2].pl[pr & 3][slot >> 1]) + (slot & 1);
        *half = static_cast<uint16_t>(rv);
        if (scur > 84) ++n_unres;  // counted: dots that needed the integer accumulator
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // 3. scores of the deferred keys from the corrected values: lane (row g, column e) sums group g of entry
  //    e with this lane's own head weights, the rows combine as in the main loop
  for (int eb = 0; eb < nent; eb += 16) {
    const int e = min(eb + l16, nent - 1);
    const float G = group_sum<HT, WBF>([&](int i) { return E[e].pl[g][i]; }, wv);
    const float tot = combine_groups(G);
    const int key = E[e].key;
    if (g == 0 && eb + l16 < nent && key < T) orow[key] = (key < limit) ? (WBF ? round_score_bf16(tot) : tot) : -INFINITY;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Shared memory of the bound-emitting variant: the key block and the per-wave norm maxima only (no
// deferred-key entries, no dot lists, no row statistics), and in the counting form each wave's counts of its
// row's lower ends (2048 buckets as 16-bit halves: a wave counts at most kKR keys).  The counts take the LDS
// of a second workgroup per CU, so the counting form is for grids of one round.
template <int KD, bool COUNT>
struct ScoresLdsBound {
  uint4 k[kKR * KD / 8];
  uint32_t cnt[COUNT ? kQW : 0][1024];
  float knorm[kKR];
  int32_t kspan[kKR];
  int32_t qspan[kQW][64];
  float qnorm[kQW][64];
  float dl[kQW][64];
  float w[kQW][64];
  uint16_t wup[kQW][64];  // |w| rounded up to bf16, for the bound MFMAs
};

// Waves per SIMD a kernel form is built for.  The non-counting bound kernel runs grids of several workgroups per
// CU: at most 168 VGPRs (three waves per SIMD) let the next workgroup start as soon as one wave per SIMD of the
// current one has finished.  The exact kernel at 16 heads of 64 dims (the drop-in shape: 4 dots per lane and tile,
// a tile one chain of dependent steps) at up to 128 VGPRs and 57 KiB of LDS holds two workgroups per CU: four waves per
// SIMD hide each other's tile latency, and one workgroup's prologue loads overlap the other's tiles.
template <int HT, int KD, bool BOUND, bool COUNT>
constexpr int score_waves() { return (BOUND && !COUNT) ? 3 : (!BOUND && HT == 1 && KD == 64) ? 4 : 1; }

template <int HT, int KD, bool WBF, bool BOUND, bool COUNT = false, bool F8 = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(score_waves<HT, KD, BOUND, COUNT>()))) void
indexer_scores_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const void *__restrict__ w,
    const float *__restrict__ qn, const int32_t *__restrict__ qsp, const float *__restrict__ kn,
    const int32_t *__restrict__ ksp, float *__restrict__ scores, int64_t S, int T, int64_t kbs, int causal,
    int64_t start_pos, int ratio, float bound_c, uint32_t *__restrict__ stats, int xcd_pk,
    float *__restrict__ bounds, float *__restrict__ kmax, uint32_t *__restrict__ row_counts,
    const float *__restrict__ ksc, float bound_r, const uint16_t *__restrict__ qsplit_rot, int qsplit_lo,
    int qsplit_hi) {
  constexpr int H = HT * 16;
  constexpr int kC = KD / 8;  // 16-byte chunks per key row
  static_assert(!BOUND || (HT == 4 && !WBF), "the bound-emitting variant is built for 64 heads, fp32 weights");
  static_assert(BOUND || !COUNT, "counts of lower ends need the bounds");
  static_assert(!F8 || BOUND, "FP8 keys are read by the bound-emitting variant");
  // per-dot interval half-widths (step_halfwidth_scale: the step-weighted magnitude sum and the step exponents, on
  // the MFMA) instead of the per-head bound_c 2^-23 ||q_h|| max ||k||: under half as wide on typical rows, so
  // under half the near ties and their exact recomputation, for three more MFMAs per 16-key tile (D = 64).  Built
  // where the registers allow it (16 heads).
  constexpr bool PDD = !BOUND && HT == 1;
  constexpr int kSteps = KD / 8;  // accumulation steps of a dot
  // F8: k points at e4m3 codes (KD bytes per row) with row scales ksc
  const uint8_t *__restrict__ k8 = reinterpret_cast<const uint8_t *>(k);
  __shared__ std::conditional_t<BOUND, ScoresLdsBound<KD, COUNT>, ScoresLds<KD, HT>> L;
  // the wave index is uniform per wave; readfirstlane lets the compiler keep the query row, the causal limit
  // and the tile loop in scalar registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  // XCD-aware placement: workgroup i of a batch slice runs on XCD i % 8 (the slice holds a multiple of 8
  // workgroups when xcd_pk > 0).  XCD j takes a (gridDim.y / Pq) x (gridDim.x / Pk) tile of (query
  // group, key block) pairs with Pk = xcd_pk, Pq = 8 / Pk, so its L2 holds Pk-th of the queries' rows and
  // Pq-th of the keys instead of every query group.
  int kblk = blockIdx.x, qgrp = blockIdx.y;
  if (xcd_pk > 0) {
    const int wg = blockIdx.y * gridDim.x + blockIdx.x, xcd = wg & 7, l = wg >> 3;
    const int gxk = gridDim.x / xcd_pk, gyq = gridDim.y / (8 / xcd_pk);
    qgrp = (xcd / xcd_pk) * gyq + l / gxk;
    kblk = (xcd % xcd_pk) * gxk + l % gxk;
  }
  const int64_t b = blockIdx.z;
  const int kb0 = kblk * kKR;
  const int nk = min(kKR, T - kb0);
  const int64_t s = static_cast<int64_t>(qgrp) * kQW + wave;
  const bool s_ok = s < S;
  const int64_t kbrow0 = b * kbs;        // first key row of batch b
  const int64_t krow0 = kbrow0 + kb0;    // first key row of this workgroup
  // A workgroup whose queries all see none of its keys (causal limits at or below the block; the last query
  // has the largest limit) only writes the mask: no staging, no statistics (uniform over the workgroup, so
  // every wave leaves before the barrier).  Its key block's norm maximum is then read by no query.
  if (causal) {
    const int64_t s_last = static_cast<int64_t>(qgrp) * kQW + kQW - 1 < S - 1 ? static_cast<int64_t>(qgrp) * kQW + kQW - 1
                                                                             : S - 1;
    if ((start_pos + s_last + 1) / ratio <= kb0) {
      if (s_ok) {
        float *orow_m = scores + (b * S + s) * T;
        for (int i = lane; i < nk; i += 64) orow_m[kb0 + i] = -INFINITY;
      }
      return;
    }
  }

  // Every prologue load is issued before the first wait (loads complete in order, so each later wait is a
  // partial one): the key statistics and this wave's query statistics and head weights, then the key
  // block, then the q fragments.  Indices are clamped into range and the values masked afterwards, so no
  // load sits behind a branch or a loop-carried wait.
  // Statistics slots are written unconditionally: threads t and t + kKR (and lanes l and l + H) load and
  // write the same entry, so no store (and no load the compiler could sink next to it) is behind a branch.
  static_assert(kKR <= kThreads && (kKR & (kKR - 1)) == 0, "key statistics: a power-of-two block");
  const int64_t qrow0 = (b * S + (s_ok ? s : 0)) * H;
  const int kt = tid & (kKR - 1);
  const bool kin = kt < nk;
  const int kst = kin ? kt : nk - 1;  // nk >= 1: the grid covers T with key blocks
  // (loads at 32-bit unsigned offsets from workgroup-uniform bases: one address instruction each)
  const float *__restrict__ knb = kn + krow0;
  const float kn_v = knb[static_cast<uint32_t>(kst)];
  const int32_t ks_v = (ksp + krow0)[static_cast<uint32_t>(kst)];
  // every wave reads the whole block's key norms (keys lane + 64 j), so that it forms the block's norm maximum,
  // and with it the interval half-widths, without waiting for the other waves
  float kn4[kKR / 64];
#pragma unroll
  for (int j = 0; j < kKR / 64; ++j) {
    const int kj = lane + 64 * j;
    kn4[j] = knb[static_cast<uint32_t>(kj < nk ? kj : nk - 1)];
  }
  const int hl = lane & (H - 1);
  const uint32_t hlu = static_cast<uint32_t>(hl);
  const float qn_v = (qn + qrow0)[hlu];
  const int32_t qs_v = (qsp + qrow0)[hlu];
  const float w_v = WBF ? bf16_to_f32((static_cast<const uint16_t *>(w) + qrow0)[hlu])
                        : (static_cast<const float *>(w) + qrow0)[hlu];
  constexpr int kKL = kKR * kC / kThreads;  // 16-byte key chunks per thread (F8: kKL / 2 loads of 16 codes)
  constexpr int kKV = F8 ? kKL / 2 : kKL;
  uint4 kv[kKV];
  float ksv[F8 ? kKV : 1];
#pragma unroll
  for (int it = 0; it < kKV; ++it) {
    const int lin = it * kThreads + tid;
    if constexpr (F8) {
      const int kr = lin / (kC / 2), ch2 = lin % (kC / 2);
      const int64_t row = krow0 + (kr < nk ? kr : nk - 1);
      kv[it] = *reinterpret_cast<const uint4 *>(k8 + row * KD + ch2 * 16);
      ksv[it] = ksc[row];
    } else {
      const int kr = lin / kC, ch = lin % kC;
      kv[it] = *reinterpret_cast<const uint4 *>(k + krow0 * KD + static_cast<uint32_t>((kr < nk ? kr : nk - 1) * KD + ch * 8));
    }
  }
  // Every wave's key-block loads are queued ahead of every q load: the memory pipeline serves a CU's loads in
  // issue order, and the waves that issued last would otherwise wait behind the others' q rows (8 x 16 KiB)
  // for their share of the key block, which the barrier below waits for.  (The scheduling barriers keep every
  // load on its side of the barrier.)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // query rows as MFMA A-fragments (rows of query 0 for a wave past S, which leaves after the barrier); the
  // barrier below waits for the key block only, so these arrive under it and the first tile's MFMAs
  // (issued in the order the first tile's MFMAs use them, k-step by k-step, so that they can start on the first
  // k-step's fragments while the rest arrive)
  uint4 qa[HT][KD / 32];
#pragma unroll
  for (int kk = 0; kk < KD / 32; ++kk)
#pragma unroll
    for (int m = 0; m < HT; ++m)
    {
      // (the exact kernel may read its q rows from two buffers, QSplit: the rotated dims from qsplit_rot)
      const uint16_t *qsrc =
          (!BOUND && qsplit_rot != nullptr && 32 * kk >= qsplit_lo && 32 * kk < qsplit_hi) ? qsplit_rot : q;
      qa[m][kk] = *reinterpret_cast<const uint4 *>(qsrc + qrow0 * KD + static_cast<uint32_t>((16 * m + l16) * KD + 32 * kk + 8 * g));
    }
  auto abs8 = [](uint4 v) {  // |x| of 8 packed bf16
    return make_uint4(v.x & 0x7FFF7FFFu, v.y & 0x7FFF7FFFu, v.z & 0x7FFF7FFFu, v.w & 0x7FFF7FFFu);
  };
  // max key norm over this workgroup's range (the error bound uses it for every key)
  L.knorm[kt] = kin ? kn_v : 0.f;
  L.kspan[kt] = kin ? ks_v : 0;
  float knm = 0.f;
#pragma unroll
  for (int j = 0; j < kKR / 64; ++j) knm = fmaxf(knm, lane + 64 * j < nk ? kn4[j] : 0.f);
  knm = wave_max_f32(knm);
  L.qspan[wave][hl] = qs_v;
  L.qnorm[wave][hl] = qn_v;
  // per-head data formed once per head (lane h), not by each of the 16 lanes that use it.  PDD (the exact kernel
  // at 16 heads): per-dot half-widths from the MFMA sum of the magnitudes, dl then holds their additive part
  L.dl[wave][hl] = PDD ? step_halfwidth_add(qn_v, knm, bound_r) : dot_halfwidth(qn_v, knm, bound_c);
  if constexpr (BOUND) L.wup[wave][hl] = bf16_abs_round_up(w_v);
  L.w[wave][hl] = w_v;
  // the workgroup's whole key block into LDS
  if constexpr (F8) {
    // one conversion form for the whole wave: the one-instruction form when every scale it holds allows it
    bool p2 = true;
#pragma unroll
    for (int it = 0; it < kKV; ++it) p2 = p2 & fp8_scale_pow2(ksv[it]);  // no short-circuit: no branches
    p2 = __builtin_amdgcn_ballot_w64(!p2) == 0ull;
    auto stage = [&](auto POW2) {
#pragma unroll
      for (int it = 0; it < kKV; ++it) {
        const int lin = it * kThreads + tid;
        const int kr = lin / (kC / 2), ch = 2 * (lin % (kC / 2));
        const uint32_t msk = kr < nk ? 0xFFFFFFFFu : 0u;
        const uint4 lo = fp8_dequant8<decltype(POW2)::value>(make_uint2(kv[it].x, kv[it].y), ksv[it]);
        const uint4 hi = fp8_dequant8<decltype(POW2)::value>(make_uint2(kv[it].z, kv[it].w), ksv[it]);
        L.k[kr * kC + (ch ^ (kr & (kC - 1)))] = make_uint4(lo.x & msk, lo.y & msk, lo.z & msk, lo.w & msk);
        L.k[kr * kC + ((ch + 1) ^ (kr & (kC - 1)))] = make_uint4(hi.x & msk, hi.y & msk, hi.z & msk, hi.w & msk);
      }
    };
    if (p2)
      stage(std::true_type{});
    else
      stage(std::false_type{});
  } else {
    // Rows past T hold copies of the last key, loaded from the clamped row: finite operands whose columns are
    // neither stored nor listed.  The 32- and 64-head kernels still zero them: with the loaded values used only by
    // the LDS stores, the compiler sinks their loads below the q loads (and the load-ordering barrier above),
    // which the mask's use of them prevents (a CPU test checks the placement in the compiled code).
    constexpr bool kMask = HT > 1;
#pragma unroll
    for (int it = 0; it < kKL; ++it) {
      const int lin = it * kThreads + tid;
      const int kr = lin / kC, ch = lin % kC;
      const uint32_t msk = (!kMask || kr < nk) ? 0xFFFFFFFFu : 0u;
      L.k[kr * kC + (ch ^ (kr & (kC - 1)))] = make_uint4(kv[it].x & msk, kv[it].y & msk, kv[it].z & msk, kv[it].w & msk);
      if constexpr (PDD) L.kstep[kr][ch] = static_cast<uint16_t>(step_exponent_pow2(kv[it]));
    }
  }
  if constexpr (COUNT) {  // this wave's lower-end counts start at zero
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<uint4 *>(L.cnt[wave])[lane + 64 * i] = make_uint4(0, 0, 0, 0);
  }
  // the only barrier (from here on every wave runs independently): LDS writes done, no wait for the q loads
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // BOUND: the block's key-norm maximum for the exact recomputation of candidate scores, which must use
  // the same interval width (every query group writes the same value)
  if constexpr (BOUND) {
    if (tid == 0) kmax[b * gridDim.x + kblk] = knm;
  }
  if (!s_ok) return;
  float wv[HT][4], dl[HT][4];
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 16 * m + 4 * g + r;
      wv[m][r] = L.w[wave][h];
      dl[m][r] = L.dl[wave][h];
    }
  // a half-width of +inf (norms that could overflow inside the MFMA): every dot of the wave is a near tie
  bool any_inf = false;
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) any_inf = any_inf || dl[m][r] == __builtin_inff();
  const bool forced = __builtin_amdgcn_ballot_w64(any_inf) != 0ull;
  // BOUND: the tile MFMAs start from -delta instead of 0, so that they return the lower interval end A - delta
  // without a subtraction, and the upper end is fl((A - delta) + 2 delta).  The accumulation model above applies
  // to any initial value: the running values now carry -delta, which adds at most 16 (2^-31 + 2^-24) delta
  // (< 2^-19 delta) to its loss; the lower end needs no fp32 rounding of its own, and the upper end's single
  // rounding loses at most 2^-24 (|A - delta| + 2 delta), as forming A + delta did.  The constant 13 still
  // covers the sum (12.07 + 0.5 + 2^-19 + the constant's 3 ulps).
  // (each -delta passes through an empty asm, so that the compiler cannot rewrite the upper end's fma in terms of
  // +delta and keep both sets of 16 registers live)
  f32x4_t negd[HT];
#pragma unroll
  for (int m = 0; m < HT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = -dl[m][r];
      asm("" : "+v"(x));
      negd[m][r] = x;
    }

  // BOUND: A-fragments holding bf16 upper bounds of |w| for the two 32-head halves.  With the relu'd
  // interval ends of a tile as B-fragments (lane (l16, g) holds heads 4g + 0..3 and 16 + 4g + 0..3 of
  // each half, exactly the k-slots 8g .. 8g + 7 of a 16x16x32 B operand), one MFMA per half sums
  // w_up * r over the 32 heads for every key, in every output row.
  uint4 wa[2] = {};
  if constexpr (BOUND) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      // heads 16 m + 4 g + (0, 1) and (2, 3) of m = 2 hh and 2 hh + 1, as packed pairs
      const uint32_t *up = reinterpret_cast<const uint32_t *>(L.wup[wave]);
      const int h0 = 16 * (2 * hh) + 4 * g, h1 = h0 + 16;
      wa[hh] = make_uint4(up[h0 / 2], up[h0 / 2 + 1], up[h1 / 2], up[h1 / 2 + 1]);
    }
  }
  const int64_t limit = causal ? (start_pos + s + 1) / ratio : INT64_MAX;
  const int limit32 = static_cast<int>(limit < INT32_MAX ? limit : INT32_MAX);  // keys are below T < 2^31
  float *orow = scores + (b * S + s) * T;
  float *urow = BOUND ? bounds + (b * S + s) * T : nullptr;
  uint32_t n_exact = 0, n_unres = 0;
  int nent = 0;
  // tiles of 16 keys; tiles at or past the causal limit are masked without MFMA work
  const int ntiles = (nk + 15) / 16;
  const int64_t lim_rel = limit - kb0;
  const int nlive = lim_rel <= 0 ? 0 : (lim_rel >= 16 * ntiles ? ntiles : static_cast<int>((lim_rel + 15) / 16));

  // PDD: accs holds V >= W + 8 M of the per-dot half-width (step_halfwidth_scale): the step-weighted magnitudes of
  // q (qw, formed once: fragment kk of this lane is step 4 kk + g, weight 2^j >= kSteps + 1 - step) against |k|,
  // then one MFMA of the step exponents: aprime holds 8 A'_s of this lane's head in k-slots 8 g .. 8 g + 7 (steps
  // 8 g ..; zeros past the last step), gathered through the wave's dot-list LDS (unused until the first flush);
  // the keys' B'_s are staged with the key block.
  uint4 qw[HT][KD / 32];
  uint4 aprime = make_uint4(0, 0, 0, 0);
  if constexpr (PDD) {
    uint16_t *sq = reinterpret_cast<uint16_t *>(L.dots[wave]);  // [16 heads][kSteps]: 8 A'_s
#pragma unroll
    for (int kk = 0; kk < KD / 32; ++kk) {
      const int st = 4 * kk + g;
      qw[0][kk] = step_weighted_q(qa[0][kk], step_weight_log2(kSteps, st));
      const uint32_t p = step_exponent_pow2(qa[0][kk]);
      sq[l16 * kSteps + st] = static_cast<uint16_t>(p == 0u ? 0u : p + (3u << 7));  // 8 A'_s: exponent + 3
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint4 t = reinterpret_cast<const uint4 *>(sq)[(l16 * kSteps + 8 * (g % (kSteps / 8))) / 8];
    aprime = g < kSteps / 8 ? t : make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // the MFMAs of 16 keys, lane l16 holding block row key_l (a tile: 16 t + l16; or rows from the deferred list)
  // (every LDS read first; PDD: the magnitude chain starts with the step exponents, so that its dependent MFMAs
  // alternate with the independent ones of the dot)
  auto tile_mfma = [&](int key_l, f32x4_t(&acc)[HT], f32x4_t(&accs)[HT]) {
    uint4 bv[KD / 32];
#pragma unroll
    for (int kk = 0; kk < KD / 32; ++kk) bv[kk] = L.k[key_l * kC + ((4 * kk + g) ^ (key_l & (kC - 1)))];
#pragma unroll
    for (int m = 0; m < HT; ++m) acc[m] = accs[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (PDD) {
      // the step exponents: lane (key row, g) reads the key's B'_s of steps 8 g .. (lanes past the last step read
      // the first ones: their A' slots are zero, so those products leave the sum unchanged)
      const uint4 bp = *reinterpret_cast<const uint4 *>(&L.kstep[key_l][8 * (g % (kSteps / 8))]);
      accs[0] = mfma16(aprime, bp, accs[0]);
    }
#pragma unroll
    for (int kk = 0; kk < KD / 32; ++kk) {
#pragma unroll
      for (int m = 0; m < HT; ++m) acc[m] = mfma16(qa[m][kk], bv[kk], acc[m]);
      if constexpr (PDD) {
        const uint4 ba = abs8(bv[kk]);
#pragma unroll
        for (int m = 0; m < HT; ++m) accs[m] = mfma16(qw[m][kk], ba, accs[m]);
      }
    }
  };
  // the same in two halves (BOUND, from -delta): the B fragments of a tile are read one tile ahead of its MFMAs
  auto tile_b = [&](int t, uint4(&bv)[KD / 32]) {
    const int key_l = 16 * t + l16;
#pragma unroll
    for (int kk = 0; kk < KD / 32; ++kk) bv[kk] = L.k[key_l * kC + ((4 * kk + g) ^ (key_l & (kC - 1)))];
  };
  auto tile_mfma_b = [&](const uint4(&bv)[KD / 32], f32x4_t(&acc)[HT]) {
#pragma unroll
    for (int m = 0; m < HT; ++m) acc[m] = negd[m];  // lower ends A - delta
#pragma unroll
    for (int kk = 0; kk < KD / 32; ++kk)
#pragma unroll
      for (int m = 0; m < HT; ++m) acc[m] = mfma16(qa[m][kk], bv[kk], acc[m]);
  };

  const float dsc = PDD ? step_halfwidth_scale(bound_r) : 0.f;
  // the exact kernel's interval test (the tile epilogue's, below) on the 16 keys of a resolution round: pl, ph and the
  // ballot of the lanes holding a near-tie dot.  (The tile epilogue keeps its own copy: sharing this lambda with
  // the bound kernels' epilogue made the compiler spill registers in their tile loop.)
  auto interval_ends = [&](const f32x4_t(&acc)[HT], const f32x4_t(&accs)[HT], uint32_t(&pl)[2 * HT],
                           uint32_t(&ph)[2 * HT]) {
    uint64_t anyr = 0;
#pragma unroll
    for (int m = 0; m < HT; ++m)
#pragma unroll
      for (int rp = 0; rp < 2; ++rp) {
        const float A0 = acc[m][2 * rp], A1 = acc[m][2 * rp + 1];
        const float d0 = PDD ? __builtin_fmaf(accs[m][2 * rp], dsc, dl[m][2 * rp]) : dl[m][2 * rp];
        const float d1 = PDD ? __builtin_fmaf(accs[m][2 * rp + 1], dsc, dl[m][2 * rp + 1]) : dl[m][2 * rp + 1];
        pl[2 * m + rp] = cvt_relu_pk(A0 - d0, A1 - d1);
        ph[2 * m + rp] = cvt_relu_pk(A0 + d0, A1 + d1);
        anyr |= __builtin_amdgcn_ballot_w64(pl[2 * m + rp] != ph[2 * m + rp]);
      }
    if (forced) {
#pragma unroll
      for (int p = 0; p < 2 * HT; ++p) {
        pl[p] = 0u;
        ph[p] = 0x7F807F80u;
      }
      anyr = ~0ull;
    }
    return anyr;
  };
  // the key mask (bit = key column) of a ballot over the four head-group rows
  auto key_mask = [](uint64_t r) { return static_cast<uint32_t>((r | (r >> 16) | (r >> 32) | (r >> 48)) & 0xFFFFull); };
  // returns the mask of this tile's keys (bit = key column) that hold a near-tie dot (in the exact kernel, before
  // the causal limit: a key past it keeps the -inf stored here); pl / ph keep the interval ends.
  // FULL (the exact kernel's tiles before its last live one): every key of the tile is in range and before the
  // causal limit, so the tile needs no per-lane key tests.  PAIR (the exact kernel): the lane's group sum is
  // returned in gsum, and store_pair combines two tiles' sums at once; otherwise the tile stores its own scores.
  auto tile_epilogue = [&](auto FC, auto FULL, auto PAIR, int t, const f32x4_t(&acc)[HT], const f32x4_t(&accs)[HT],
                           uint32_t(&pl)[2 * HT], uint32_t(&ph)[2 * HT], float &gsum) {
    const bool fcd = decltype(FC)::value;
    constexpr bool full = decltype(FULL)::value;
    const int key_l = 16 * t + l16;
    const int key = kb0 + key_l;
    const bool kvalid = full || key_l < nk;
    // interval test: RNE(A - delta) == RNE(A + delta) (after ReLU) <=> the exact dot rounds to the same
    // relu'd bf16 value; pl holds that value for the head sum
    uint64_t anyr = 0;
#pragma unroll
    for (int m = 0; m < HT; ++m)
#pragma unroll
      for (int rp = 0; rp < 2; ++rp) {
        const float A0 = acc[m][2 * rp], A1 = acc[m][2 * rp + 1];
        if constexpr (BOUND) {  // A0, A1 are already the lower ends A - delta
          const float n0 = negd[m][2 * rp], n1 = negd[m][2 * rp + 1];
          pl[2 * m + rp] = cvt_relu_pk(A0, A1);
          ph[2 * m + rp] = cvt_relu_pk(__builtin_fmaf(-2.f, n0, A0), __builtin_fmaf(-2.f, n1, A1));
        } else {
          const float d0 = PDD ? __builtin_fmaf(accs[m][2 * rp], dsc, dl[m][2 * rp]) : dl[m][2 * rp];
          const float d1 = PDD ? __builtin_fmaf(accs[m][2 * rp + 1], dsc, dl[m][2 * rp + 1]) : dl[m][2 * rp + 1];
          pl[2 * m + rp] = cvt_relu_pk(A0 - d0, A1 - d1);
          ph[2 * m + rp] = cvt_relu_pk(A0 + d0, A1 + d1);
        }
        anyr |= __builtin_amdgcn_ballot_w64(pl[2 * m + rp] != ph[2 * m + rp]);
      }
    if (fcd) {  // wave-uniform and rare: A may not even be finite; the exact values replace everything
#pragma unroll
      for (int p = 0; p < 2 * HT; ++p) {
        pl[p] = 0u;
        ph[p] = 0x7F807F80u;
      }
      anyr = ~0ull;
    }
    // canonical head sum of this lane's group, then ((G0+G1)+(G2+G3)) across the rows
    float G = 0.f;
    if constexpr (WBF) {
      G = group_sum<HT, WBF>([&](int i) { return pl[i]; }, wv);
    } else {
#pragma unroll
      for (int m = 0; m < HT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t p2 = pl[2 * m + (r >> 1)];
          const float rv = (r & 1) ? unpack_hi(p2) : unpack_lo(p2);
          G = __builtin_fmaf(rv, wv[m][r], G);
        }
    }
    if constexpr (BOUND) {
      // the next tile's 16 MFMAs (issued before this epilogue, in the same basic block) spread over the interval
      // test and the head sum, one per 6 VALU instructions: the wave keeps issuing VALU work while the matrix
      // core runs, instead of stalling on 16 back-to-back MFMAs
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
      }
    }
    float tot = 0.f, outv = 0.f;
    if constexpr (decltype(PAIR)::value) {
      gsum = G;
    } else {
      tot = combine_groups(G);
      outv = WBF ? round_score_bf16(tot) : tot;
      if (g == 0 && kvalid) orow[key] = (full || key < limit32) ? outv : -INFINITY;
    }
    // keys past T are not stored and, in the exact kernel, keys past the causal limit are -inf: neither is deferred
    // (the bound kernel stores bound 0 past the limit, below)
    if constexpr (!full) anyr &= __builtin_amdgcn_ballot_w64(BOUND ? kvalid : (kvalid && key < limit32));
    const uint32_t km = key_mask(anyr);
    if constexpr (BOUND) {
      // |exact score - tot| <= sum_h |w_h| (ph_h - pl_h) + (rounding of the canonical sum: 38 roundings of
      // at most 2^-24 of sum_h |w_h| ph_h, < 2^-18 of it) <= dph - dpl + 2^-16 (dph + dpl), dph / dpl the
      // MFMA sums of w_up * ph / pl (64 nonnegative exact products in 8 accumulation steps: relative error
      // below (8 + 8) 2^-24 < 2^-19 by the step model of dot_halfwidth, the 2^-100 term covering subnormal
      // operands).  The 2^-21 |tot| term lets tot -/+ bound be rounded to nearest and stay a bound.  Keys
      // without a near-tie dot have bound 0 (tot is exact).
      f32x4_t dph = f32x4_t{0.f, 0.f, 0.f, 0.f}, dpl = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        dph = mfma16(wa[hh], make_uint4(ph[4 * hh], ph[4 * hh + 1], ph[4 * hh + 2], ph[4 * hh + 3]), dph);
        dpl = mfma16(wa[hh], make_uint4(pl[4 * hh], pl[4 * hh + 1], pl[4 * hh + 2], pl[4 * hh + 3]), dpl);
      }
      float u = (dph[0] - dpl[0]) + 0x1p-16f * (dph[0] + dpl[0]) + 0x1p-21f * fabsf(tot) + 0x1p-100f;
      if (fcd) u = __builtin_inff();  // score 0 with an infinite bound: always recomputed
      const bool live_key = kvalid && key < limit32;
      const float us = (live_key && ((km >> l16) & 1u)) ? u : 0.f;
      if (g == 0 && kvalid) urow[key] = us;
      // the row's threshold histogram: first 11-bit digit of the lower end's key, counted for the valid columns
      // (the same arithmetic as the stored score and bound give)
      if (COUNT && g == 0 && live_key) {
        const uint32_t kk = score_key(us > 0.f ? outv - us : outv);
        if (kk != 0u) atomicAdd(&L.cnt[wave][kk >> 22], 1u << ((kk >> 17) & 16u));
      }
    }
    return km;
  };

  // software pipeline: the MFMAs of the next tile are in flight during the current tile's epilogue.
  f32x4_t acc[HT], nxt[HT];
  if constexpr (BOUND) {
    // no deferred keys: two tiles per iteration, alternating the accumulator sets (no copy between them) and
    // the B-fragment sets (read one tile ahead).  The MFMAs and reads past the last live tile repeat that tile
    // (results unused), so that no branch separates them from the epilogue they are interleaved with.
    auto run = [&](auto FC) {
      uint4 ba[KD / 32], bb[KD / 32];
      const int last = nlive - 1;
      tile_b(0, ba);
      tile_mfma_b(ba, acc);
      tile_b(1 < nlive ? 1 : last, bb);
      for (int t = 0; t < nlive; t += 2) {
        uint32_t pl[2 * HT], ph[2 * HT];
        tile_mfma_b(bb, nxt);
        tile_b(t + 2 < nlive ? t + 2 : last, ba);
        float gs;
        (void)tile_epilogue(FC, std::false_type{}, std::false_type{}, t, acc, acc, pl, ph, gs);
        if (t + 1 >= nlive) break;
        tile_mfma_b(ba, acc);
        tile_b(t + 3 < nlive ? t + 3 : last, bb);
        (void)tile_epilogue(FC, std::false_type{}, std::false_type{}, t + 1, nxt, nxt, pl, ph, gs);
      }
    };
    if (nlive > 0) {
      if (forced)
        run(std::true_type{});
      else
        run(std::false_type{});
    }
  }
  if constexpr (!BOUND) {
    // the exact kernel: the tile loop only lists the keys holding a near-tie dot (their block rows, in LDS); the
    // listed keys are resolved after it.  Nothing of the recomputation is live in the loop, so the loop keeps its
    // pipeline in few registers.  The next tile's MFMAs past the last live tile repeat that tile (results unused).
    // Two tiles per iteration alternate the accumulator sets (no copies between them); the loop is built twice,
    // for forced waves (every key listed) and the others, so that the tile epilogue carries no select for it.
    f32x4_t accs[HT], nxts[HT];
    uint8_t *klist = L.klist[wave];
    int nlist = 0;
    // Tiles before the last live one are full (every key in range and before the limit).
    auto epilogue = [&](auto FC, auto FULL, auto PAIR, int t, const f32x4_t(&a)[HT], const f32x4_t(&as)[HT]) {
      uint32_t pl[2 * HT], ph[2 * HT];
      float gs = 0.f;
      const uint32_t km = tile_epilogue(FC, FULL, PAIR, t, a, as, pl, ph, gs);
      if (km != 0u) {  // wave-uniform
        if (g == 0 && ((km >> l16) & 1u))
          klist[nlist + __builtin_popcount(km & ((1u << l16) - 1u))] = static_cast<uint8_t>(16 * t + l16);
        nlist += __builtin_popcount(km);
      }
      return gs;
    };
    // The scores of tiles t and t + 1 from their lanes' group sums ga, gb: ((G0 + G1) + (G2 + G3)) of both tiles
    // with one exchange of each kind (combine_groups with two different registers in place of one copied twice):
    // after the row-pair swap, rows 0 / 2 hold tile t's pair sums and rows 1 / 3 tile t + 1's; after the half swap
    // row 0 holds tile t's score and row 1 tile t + 1's.  PB: tile t + 1 is the last live tile (key tests).
    auto store_pair = [&](auto PB, int t, float ga, float gb) {
      float a = ga, b = gb;
      asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
      float c = a + b, d = c;
      asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(c), "+v"(d));
      const float tot = c + d;
      const float outv = WBF ? round_score_bf16(tot) : tot;
      const int key_l = 16 * (t + (g & 1)) + l16;
      if constexpr (decltype(PB)::value) {
        if (g == 0 || (g == 1 && key_l < nk)) orow[kb0 + key_l] = (g == 0 || kb0 + key_l < limit32) ? outv : -INFINITY;
      } else {
        if (g < 2) orow[static_cast<uint32_t>(kb0 + key_l)] = outv;
      }
    };
    const int last = nlive - 1;
    if (nlive > 0 && !forced) {
      const std::true_type full, pair;
      const std::false_type fc, partial, single;
      tile_mfma(l16, acc, accs);
      int t = 0;
      for (; t + 2 <= last; t += 2) {
        tile_mfma(16 * (t + 1) + l16, nxt, nxts);
        const float ga = epilogue(fc, full, pair, t, acc, accs);
        tile_mfma(16 * (t + 2) + l16, acc, accs);
        const float gb = epilogue(fc, full, pair, t + 1, nxt, nxts);
        store_pair(std::false_type{}, t, ga, gb);
      }
      if (t < last) {
        tile_mfma(16 * last + l16, nxt, nxts);
        const float ga = epilogue(fc, full, pair, t, acc, accs);
        const float gb = epilogue(fc, partial, pair, last, nxt, nxts);
        store_pair(std::true_type{}, t, ga, gb);
      } else {
        (void)epilogue(fc, partial, single, last, acc, accs);
      }
    } else if (nlive > 0) {
      // a forced wave lists every key (its interval ends are not used)
      for (int t = 0; t < nlive; ++t) (void)epilogue(std::true_type{}, std::false_type{}, std::false_type{}, t, acc, accs);
    }
    // resolution, 16 listed keys at a time: the same MFMAs and interval test on their rows (the same operands, so
    // the same interval ends)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (HT == 1) {
      // 16 heads: each round keeps its 16 keys' interval ends in registers (lane (g, l16): heads 4 g .. 4 g + 3 of
      // key l16), lists the round's near-tie dots (lane and head bit, 16 bits each; at most 256) in the wave's dot list,
      // computes them exactly 16 at a time, patches the exact relu'd values (through the list's patch slots, one
      // per lane and head bit) into its own ends and stores the round's scores.
      const QSplit qsp{qsplit_rot, qsplit_lo, qsplit_hi};
      // a round holds at most 16 keys x 16 heads = 256 near-tie dots: [0, 256) the list, [256, 512) the patches
      static_assert(2 * 256 * sizeof(uint16_t) <= sizeof(L.dots[0]), "dot list and patches of one round");
      uint16_t *Dl = reinterpret_cast<uint16_t *>(L.dots[wave]);
      uint16_t *Pt = Dl + 256;
      const int dq = lane >> 2, sub = lane & 3;
      for (int base = 0; base < nlist; base += 16) {
        const int key_l = klist[min(base + l16, nlist - 1)];
        tile_mfma(key_l, acc, accs);
        uint32_t pl[2], ph[2];
        (void)interval_ends(acc, accs, pl, ph);
        // this lane's near-tie dots: bit b = head 4 g + b (half b & 1 of pl[b >> 1]); lanes past the list none
        uint32_t m = 0;
        if (base + l16 < nlist) {
          const uint32_t d0 = pl[0] ^ ph[0], d1 = pl[1] ^ ph[1];
          m = ((d0 & 0xFFFFu) ? 1u : 0u) | ((d0 >> 16) ? 2u : 0u) | ((d1 & 0xFFFFu) ? 4u : 0u) | ((d1 >> 16) ? 8u : 0u);
        }
        uint32_t nd_u;
        uint32_t pos = wave_excl_scan_bits<3>(static_cast<uint32_t>(__builtin_popcount(m)), nd_u);
        for (uint32_t mm = m; mm != 0u; mm &= mm - 1u) Dl[pos++] = static_cast<uint16_t>((lane << 2) | __builtin_ctz(mm));
        n_exact += nd_u;
        const int nd = static_cast<int>(nd_u);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int b0 = 0; b0 < nd; b0 += 16) {
          // the quad's dot (idle quads repeat the last one; the result is identical): lane sl's head bit
          const int dcur = Dl[min(b0 + dq, nd - 1)];
          const int sl = dcur >> 2;
          const int h = 4 * (sl >> 4) + (dcur & 3);
          const int kl = klist[base + (sl & 15)];
          int scur;
          const uint16_t r = quad_exact_dot<HT, KD>(L, wave, sub, h, kl, q, qsp, qa, qrow0, scur);
          if (sub == 0 && b0 + dq < nd) {
            Pt[dcur] = (r & 0x8000) ? 0u : r;  // ReLU (also maps -0 to +0)
            if (scur > 84) ++n_unres;  // counted: dots that needed the integer accumulator
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (m != 0u) {
#pragma unroll
          for (int bit = 0; bit < 4; ++bit)
            if ((m >> bit) & 1u) {
              const uint32_t v = Pt[(lane << 2) | bit];
              uint32_t &w2 = pl[bit >> 1];
              w2 = (bit & 1) ? ((w2 & 0xFFFFu) | (v << 16)) : ((w2 & 0xFFFF0000u) | v);
            }
        }
        // the round's scores from the patched values (every listed key is in range and before the causal limit)
        const float G = group_sum<HT, WBF>([&](int i) { return pl[i]; }, wv);
        const float tot = combine_groups(G);
        if (g == 0 && base + l16 < nlist) orow[static_cast<uint32_t>(kb0 + key_l)] = WBF ? round_score_bf16(tot) : tot;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else {
      // all four groups' ends of each key saved as a deferred entry, and the entries' near-tie dots computed
      // exactly and their scores rewritten whenever another 16 could overflow the entries
      for (int base = 0; base < nlist; base += 16) {
        const int key_l = klist[min(base + l16, nlist - 1)];
        tile_mfma(key_l, acc, accs);
        uint32_t pl[2 * HT], ph[2 * HT];
        // every listed key is in range and before the causal limit; lanes past the list repeat its last key
        const uint32_t km = key_mask(interval_ends(acc, accs, pl, ph) &
                                     __builtin_amdgcn_ballot_w64(base + l16 < nlist));
        if ((km >> l16) & 1u) {
          const int e = nent + __builtin_popcount(km & ((1u << l16) - 1u));
          KeyEntry<HT> &en = L.ent[wave][e];
#pragma unroll
          for (int p = 0; p < 2 * HT; ++p) {
            en.pl[g][p] = pl[p];
            en.ph[g][p] = ph[p];
          }
          if (g == 0) en.key = kb0 + key_l;
        }
        nent += __builtin_popcount(km);
        if (nent + 16 > kEntCap || base + 16 >= nlist) {
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          if (nent > 0)
            flush_entries<HT, KD, WBF>(L, wave, lane, nent, q, qa, qrow0, orow, limit, T, kb0, wv, n_exact, n_unres,
                                       QSplit{qsplit_rot, qsplit_lo, qsplit_hi});
          nent = 0;
        }
      }
    }
  }
  // masked tiles (at or past the causal limit); the exact kernel stores with every lane (the bound kernel keeps
  // its tile form, which its register allocation was tuned with)
  if constexpr (BOUND) {
    for (int t = nlive; t < ntiles; ++t) {
      const int key_l = 16 * t + l16;
      if (g == 0 && key_l < nk) orow[kb0 + key_l] = -INFINITY;
    }
  } else {
    for (int key_l = 16 * nlive + lane; key_l < nk; key_l += 64) orow[static_cast<uint32_t>(kb0 + key_l)] = -INFINITY;
  }
  if constexpr (COUNT) {
    // the wave's counts into its row's histogram (only the nonzero buckets: a block of 256 keys fills a few
    // dozen of the 2048)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint32_t *hrow = row_counts + (b * S + s) * 2048;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int wd = lane + 64 * i;
      const uint32_t v = L.cnt[wave][wd];
      if (v & 0xFFFFu) atomicAdd(&hrow[2 * wd], v & 0xFFFFu);
      if (v >> 16) atomicAdd(&hrow[2 * wd + 1], v >> 16);
    }
  }
  if (stats != nullptr) {
    if (lane == 0 && n_exact) atomicAdd(&stats[0], n_exact);
    if (n_unres) atomicAdd(&stats[1], n_unres);
  }
}

template <int HT, int KD>
int launch_scores_ht(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                     const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B, int64_t S,
                     int64_t T, int64_t kbs, int causal, int64_t start_pos, int ratio, float bound_c, uint32_t *stats,
                     float *bounds, float *kmax, uint32_t *row_counts, const float *ksc, hipStream_t stream,
                     const QSplit *qsplit) {
  const QSplit qs = qsplit != nullptr ? *qsplit : QSplit{nullptr, 0, 0};
  dim3 grid(static_cast<unsigned>(ceil_div(T, kKR)), static_cast<unsigned>(ceil_div(S, kQW)),
            static_cast<unsigned>(B));
  const float bound_r = bound_c / score_bound_c(KD);  // the per-dot half-widths' scale (16-head exact kernel)
  // XCD tiling (Pq x Pk = 8) that minimises the L2 fills: each query group's rows are read by Pk XCDs,
  // each key block by Pq; 0 keeps the launch order (slice not a multiple of 8 or no tiling divides it)
  int xcd_pk = 0;
  if ((static_cast<int64_t>(grid.x) * grid.y) % 8 == 0) {
    const double qbytes = static_cast<double>(S) * 16 * HT * KD, kbytes = static_cast<double>(T) * KD;  // either format
    double best = 0.0;
    for (int pk = 1; pk <= 8; pk *= 2) {
      const int pq = 8 / pk;
      if (grid.x % pk != 0 || grid.y % pq != 0) continue;
      const double cost = qbytes * pk + kbytes * pq;
      if (xcd_pk == 0 || cost < best) {
        best = cost;
        xcd_pk = pk;
      }
    }
  }
  if (ksc != nullptr && bounds == nullptr)
    return fail(KS_ERR_INVALID, "indexer scores: FP8 keys need the bound-emitting kernel");
  if (bounds != nullptr && ksc != nullptr) {
    if constexpr (HT == 4 && KD == 128) {
      if (w_bf16) return fail(KS_ERR_INVALID, "indexer scores: score bounds need fp32 weights");
      if (kmax == nullptr) return fail(KS_ERR_INVALID, "indexer scores: score bounds need the kmax buffer");
      if (row_counts != nullptr) {
        hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, false, true, true, true>), grid, dim3(kThreads), 0, stream, q,
                           k, w, qn, qsp, kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio,
                           bound_c, stats, xcd_pk, bounds, kmax, row_counts, ksc, bound_r, qs.rot, qs.lo, qs.hi);
      } else {
        hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, false, true, false, true>), grid, dim3(kThreads), 0, stream,
                           q, k, w, qn, qsp, kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio,
                           bound_c, stats, xcd_pk, bounds, kmax, nullptr, ksc, bound_r, qs.rot, qs.lo, qs.hi);
      }
    } else {
      return fail(KS_ERR_INVALID, "indexer scores: FP8 keys need H = 64 and D = 128");
    }
  } else if (bounds != nullptr) {
    if constexpr (HT == 4) {
      if (w_bf16) return fail(KS_ERR_INVALID, "indexer scores: score bounds need fp32 weights");
      if (kmax == nullptr) return fail(KS_ERR_INVALID, "indexer scores: score bounds need the kmax buffer");
      if (row_counts != nullptr) {
        hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, false, true, true>), grid, dim3(kThreads), 0, stream, q, k, w,
                           qn, qsp, kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c,
                           stats, xcd_pk, bounds, kmax, row_counts, nullptr, bound_r, qs.rot, qs.lo, qs.hi);
      } else {
        hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, false, true, false>), grid, dim3(kThreads), 0, stream, q, k,
                           w, qn, qsp, kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c,
                           stats, xcd_pk, bounds, kmax, nullptr, nullptr, bound_r, qs.rot, qs.lo, qs.hi);
      }
    } else {
      return fail(KS_ERR_INVALID, "indexer scores: score bounds need H = 64");
    }
  } else if (w_bf16) {
    hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, true, false>), grid, dim3(kThreads), 0, stream, q, k, w, qn, qsp,
                       kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c, stats, xcd_pk,
                       nullptr, nullptr, nullptr, nullptr, bound_r, qs.rot, qs.lo, qs.hi);
  } else {
    hipLaunchKernelGGL((indexer_scores_kernel<HT, KD, false, false>), grid, dim3(kThreads), 0, stream, q, k, w, qn,
                       qsp, kn, ksp, scores, S, static_cast<int>(T), kbs, causal, start_pos, ratio, bound_c, stats,
                       xcd_pk, nullptr, nullptr, nullptr, nullptr, bound_r, qs.rot, qs.lo, qs.hi);
  }
  KS_CHECK_LAUNCH("indexer_scores_kernel");
  return KS_OK;
}

template <int KD>
int launch_scores_d(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                    const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B, int64_t S,
                    int64_t H, int64_t T, int64_t kbs, int causal, int64_t start_pos, int ratio, float bound_c,
                    uint32_t *stats, float *bounds, float *kmax, uint32_t *row_counts, const float *ksc,
                    hipStream_t stream, const QSplit *qsplit) {
  switch (H) {
    case 16:
      return launch_scores_ht<1, KD>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos,
                                     ratio, bound_c, stats, bounds, kmax, row_counts, ksc, stream, qsplit);
    case 32:
      return launch_scores_ht<2, KD>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos,
                                     ratio, bound_c, stats, bounds, kmax, row_counts, ksc, stream, qsplit);
    case 64:
      return launch_scores_ht<4, KD>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, T, kbs, causal, start_pos,
                                     ratio, bound_c, stats, bounds, kmax, row_counts, ksc, stream, qsplit);
    default:
      return fail(KS_ERR_INVALID, "indexer scores: H=%lld, supported: 16, 32, 64", (long long)H);
  }
}

}  // namespace

bool scores_count_rows(int64_t B, int64_t S, int64_t T) {
  return ceil_div(T, kKR) * ceil_div(S, kQW) * B <= kScoreCountGrid;
}

int launch_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, const float *qn,
                          const int32_t *qsp, const float *kn, const int32_t *ksp, float *scores, int64_t B,
                          int64_t S, int64_t H, int64_t D, int64_t T, int64_t kbs, int causal, int64_t start_pos,
                          int ratio, float bound_c, uint32_t *stats, hipStream_t stream, float *bounds,
                          float *kmax, uint32_t *row_counts, const float *ksc, const QSplit *qsplit) {
  if (D == 128)
    return launch_scores_d<128>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, H, T, kbs, causal, start_pos, ratio,
                                bound_c, stats, bounds, kmax, row_counts, ksc, stream, qsplit);
  if (D == 64)
    return launch_scores_d<64>(q, k, w, w_bf16, qn, qsp, kn, ksp, scores, B, S, H, T, kbs, causal, start_pos, ratio,
                               bound_c, stats, bounds, kmax, row_counts, ksc, stream, qsplit);
  return fail(KS_ERR_INVALID, "indexer scores: D=%lld, supported: 64, 128", (long long)D);
}

}  // namespace ks

namespace {
int check_scores_args(const uint16_t *q, const uint16_t *k, const void *w, const float *qn, const int32_t *qsp,
                      const float *kn, const int32_t *ksp, float *scores, int64_t B, int64_t S, int64_t H, int64_t D,
                      int64_t T, int64_t kbs, int32_t ratio, int64_t start_pos) {
  KS_CHECK_ARG(D == 128 || D == 64, "ks_indexer_scores: D=%lld, the kernel is built for head_dim 64 and 128",
               (long long)D);
  KS_CHECK_ARG(H == 16 || H == 32 || H == 64, "ks_indexer_scores: H=%lld must be 16, 32 or 64", (long long)H);
  KS_CHECK_ARG(B >= 0 && S >= 0, "ks_indexer_scores: negative B or S");
  KS_CHECK_ARG(B < 65536 && S < (int64_t(1) << 24), "ks_indexer_scores: B or S too large");
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
  return ks::launch_indexer_scores(q, k, w, w_bf16 ? 1 : 0, q_norm, q_span, k_norm, k_span, scores, B, S, H, D,
                                   T, k_batch_stride, causal ? 1 : 0, start_pos, ratio, ks::score_bound_c(D), nullptr,
                                   static_cast<hipStream_t>(stream));
}

// Diagnostic (not part of the public header): the interval constant the public entry points use for 128-dim
// dots, and for D-dimensional ones.
extern "C" float ks_dbg_score_bound_c(void) { return ks::kScoreBoundC; }
extern "C" float ks_dbg_score_bound_c_d(int64_t D) { return ks::score_bound_c(D); }

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
  return ks::launch_indexer_scores(q, k, w, w_bf16 ? 1 : 0, q_norm, q_span, k_norm, k_span, scores, B, S, H, D,
                                   T, k_batch_stride, causal ? 1 : 0, start_pos, ratio, bound_c, stats,
                                   static_cast<hipStream_t>(stream));
}

// Diagnostic variant of the bounded score kernel (not part of the public header), for timing it alone:
// as ks_dbg_indexer_scores with fp32 weights, 64 heads and D = 128, plus the per-score bounds [B, S, T],
// the key-block norm maxima [B, ceil(T / 256)] and the bounded selection's workspace part
// (ks_dbg_topk_bounded_slots(B S, T) 64-bit slots).  Where the fused entry counts the rows in the score
// kernel (ks::scores_count_rows), so does this one, into part's count region, which must then be zero.
extern "C" int ks_dbg_indexer_scores_bounded(const uint16_t *q, const uint16_t *k, const float *w,
                                             const float *q_norm, const int32_t *q_span, const float *k_norm,
                                             const int32_t *k_span, float *scores, float *bounds, float *kmax,
                                             uint64_t *part, int64_t B, int64_t S, int64_t T, int32_t causal,
                                             int64_t start_pos, void *stream) {
  ks::last_error().clear();
  int rc = check_scores_args(q, k, w, q_norm, q_span, k_norm, k_span, scores, B, S, 64, 128, T, T, 1, start_pos);
  if (rc != KS_OK) return rc;
  KS_CHECK_ARG(bounds && kmax && part, "ks_dbg_indexer_scores_bounded: null pointer");
  KS_CHECK_ARG(T <= 32768, "ks_dbg_indexer_scores_bounded: T <= 32768");
  if (B * S == 0) return KS_OK;
  return ks::launch_indexer_scores(q, k, w, 0, q_norm, q_span, k_norm, k_span, scores, B, S, 64, 128, T, T,
                                   causal ? 1 : 0, start_pos, 1, ks::kScoreBoundC, nullptr,
                                   static_cast<hipStream_t>(stream), bounds, kmax,
                                   ks::scores_count_rows(B, S, T) ? ks::topk_bounded_counts(part, B * S, T) : nullptr);
}
