/*
 * ks_oracle.c — CPU oracle for the indexer score path.  TEST INFRASTRUCTURE ONLY:
 * used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker; never part of the product path.
 *
 * It restates baseline/indexer.py:176-193 (einsum -> relu -> * weights -> head sum
 * -> causal mask) in the canonical arithmetic order that the HIP kernels promise
 * bit for bit (see include/kswift.h, ks_indexer_scores):
 *   d_h   = exact real dot product of the bf16 vectors, rounded ONCE to bf16 (RNE)
 *           (the einsum's bf16 output, baseline/indexer.py:176-180, with the fp32
 *           accumulation order pinned to "exact");
 *   r_h   = max(d_h, +0)                                   (relu_, :182)
 *   fp32 weights: G_g = fmaf(r_h, w_h, G_g)               (:182-183)
 *   bf16 weights: G_g = G_g + bf16(r_h * w_h)
 *   heads split into 4 groups g = (h/4) % 4, each summed in increasing h from +0;
 *   score = (G_0 + G_1) + (G_2 + G_3)  [rounded to bf16 for bf16 weights];
 *   causal: key t visible to query s iff t < (start_pos + s + 1) / ratio (:185-193,
 *   generalised from start_pos == 0), else -inf.
 *
 * The exact dot uses integer arithmetic: every bf16 value is m * 2^e with |m| < 256,
 * every product an integer (|.| < 2^16) times a power of two; the sum is accumulated
 * exactly in a 128-bit integer when the products' exponent spread allows, else in a
 * 12-limb two's-complement big integer, and rounded once to bf16.
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off -shared -fPIC (oracle/build.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef __int128 i128;

static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* bf16 bits -> (signed integer significand m, exponent e) with value m * 2^e.
   Returns 0 for zero (m = 0).  Inf/NaN are not expected (caller validates). */
static inline void bf_decompose(uint16_t h, int32_t *m, int32_t *e) {
  int32_t ex = (h >> 7) & 0xff;
  int32_t fr = h & 0x7f;
  int32_t mm;
  if (ex == 0) {
    mm = fr;          /* subnormal: fr * 2^-133 */
    *e = -133;
  } else {
    mm = fr | 0x80;   /* normal: (128 + fr) * 2^(ex - 127 - 7) */
    *e = ex - 134;
  }
  *m = (h & 0x8000) ? -mm : mm;
}

/* ---- round an exact value  V = mag * 2^e2 (mag > 0 given as a bit-scanned big
 * number) to bf16 RNE.  We pass the value as: top 64 significant bits `hi64`
 * (MSB set), exponent of hi64's LSB `e_lsb`, and a sticky flag for any nonzero
 * bits below hi64. */
static uint16_t round_to_bf16(int neg, uint64_t hi64, int e_lsb, int sticky) {
  /* value = hi64 * 2^e_lsb (+ sticky), hi64 has bit 63 set.
     Unbiased exponent of the leading bit: E = e_lsb + 63. */
  int E = e_lsb + 63;
  uint16_t sign = neg ? 0x8000 : 0;
  if (E > 127) return sign | 0x7f80; /* overflow -> inf */
  /* Number of significand bits kept: normal -> 8 (incl. hidden), with leading bit at 2^E.
     For subnormal results (E < -126) the LSB is fixed at 2^-133. */
  int lsb_exp = (E >= -126) ? (E - 7) : -133;
  int drop = lsb_exp - e_lsb; /* number of low bits of hi64 dropped (>= 56 normally) */
  uint64_t kept, rem_half, rem_low;
  if (drop >= 64) {
    /* everything is below the LSB: only round bit / sticky from hi64 */
    kept = 0;
    if (drop == 64) {
      rem_half = hi64 >> 63;
      rem_low = (hi64 << 1) != 0 || sticky;
    } else {
      rem_half = 0;
      rem_low = 1;
    }
  } else {
    kept = hi64 >> drop;
    rem_half = (hi64 >> (drop - 1)) & 1;
    uint64_t mask = (drop - 1 == 0) ? 0 : ((drop - 1 >= 64) ? ~0ull : ((1ull << (drop - 1)) - 1));
    rem_low = ((hi64 & mask) != 0) || sticky;
  }
  /* RNE */
  if (rem_half && (rem_low || (kept & 1))) kept += 1;
  /* kept is the significand at lsb_exp. Re-normalise. */
  if (kept == 0) return sign; /* underflow to zero */
  int32_t exp_field;
  uint32_t frac;
  if (lsb_exp == -133 && kept < 0x80) {
    exp_field = 0;
    frac = (uint32_t)kept;
  } else {
    /* kept in [0x80, 0x100]; 0x100 means carry into next binade */
    int e_lead = lsb_exp + 7;
    if (kept >= 0x100) {
      kept >>= 1;
      e_lead += 1;
    }
    if (e_lead > 127) return sign | 0x7f80;
    exp_field = e_lead + 127;
    frac = (uint32_t)kept & 0x7f;
  }
  return sign | (uint16_t)(exp_field << 7) | (uint16_t)frac;
}

/* Big two's-complement accumulator: NL 64-bit limbs, bit 0 of limb 0 = 2^BIG_LSB. */
#define NL 12
#define BIG_LSB (-300)

typedef struct {
  uint64_t l[NL];
} big_t;

static void big_add_shifted(big_t *a, int64_t v, int pos) {
  /* add v * 2^pos (pos >= 0 relative to BIG_LSB) */
  int limb = pos >> 6, off = pos & 63;
  uint64_t lo, hi, ext;
  if (v >= 0) {
    ext = 0;
  } else {
    ext = ~0ull;
  }
  /* 128-bit shifted value */
  unsigned __int128 w = (unsigned __int128)(__int128)v << off;
  lo = (uint64_t)w;
  hi = (uint64_t)(w >> 64);
  unsigned __int128 carry = 0;
  for (int i = limb; i < NL; ++i) {
    uint64_t addend = (i == limb) ? lo : (i == limb + 1) ? hi : ext;
    unsigned __int128 s = (unsigned __int128)a->l[i] + addend + carry;
    a->l[i] = (uint64_t)s;
    carry = s >> 64;
  }
}

static uint16_t big_round(const big_t *a0) {
  big_t a = *a0;
  int neg = (a.l[NL - 1] >> 63) & 1;
  if (neg) { /* negate */
    unsigned __int128 c = 1;
    for (int i = 0; i < NL; ++i) {
      unsigned __int128 s = (unsigned __int128)(~a.l[i]) + c;
      a.l[i] = (uint64_t)s;
      c = s >> 64;
    }
  }
  int top = -1;
  for (int i = NL - 1; i >= 0; --i)
    if (a.l[i]) { top = i; break; }
  if (top < 0) return 0; /* exact zero -> +0 */
  int lz = __builtin_clzll(a.l[top]);
  int msb = top * 64 + (63 - lz); /* bit index of leading one */
  /* extract 64 bits ending at msb */
  uint64_t hi64 = 0;
  int sticky = 0;
  int start = msb - 63; /* bit index of hi64's LSB (may be negative) */
  for (int b = 0; b < 64; ++b) {
    int idx = start + b;
    if (idx < 0) continue;
    if ((a.l[idx >> 6] >> (idx & 63)) & 1) hi64 |= 1ull << b;
  }
  for (int idx = 0; idx < start; ++idx)
    if ((a.l[idx >> 6] >> (idx & 63)) & 1) { sticky = 1; break; }
  if (start < 0) {
    /* fewer than 64 bits: left-align */
    hi64 <<= 0; /* already positioned: bits below index 0 are zero */
  }
  return round_to_bf16(neg, hi64, start + BIG_LSB, sticky);
}

/* Exact dot of two bf16 vectors, rounded once to bf16 (RNE). */
uint16_t ko_dot_exact_bf16(const uint16_t *a, const uint16_t *b, int64_t n) {
  int32_t ma[4096], mb[4096];
  int32_t ee[4096];
  if (n > 4096) return 0x7fc0; /* unsupported length: NaN marker */
  int cnt = 0, emin = 1 << 30, emax = -(1 << 30);
  for (int64_t i = 0; i < n; ++i) {
    int32_t m1, e1, m2, e2;
    bf_decompose(a[i], &m1, &e1);
    bf_decompose(b[i], &m2, &e2);
    if (m1 == 0 || m2 == 0) continue;
    ma[cnt] = m1;
    mb[cnt] = m2;
    ee[cnt] = e1 + e2;
    if (ee[cnt] < emin) emin = ee[cnt];
    if (ee[cnt] > emax) emax = ee[cnt];
    ++cnt;
  }
  if (cnt == 0) return 0;
  if (emax - emin <= 96) {
    /* |sum| < cnt * 2^16 * 2^(emax-emin) <= 2^(12+16+96) < 2^127 */
    i128 acc = 0;
    for (int i = 0; i < cnt; ++i) acc += (i128)((int64_t)ma[i] * mb[i]) << (ee[i] - emin);
    if (acc == 0) return 0;
    int neg = acc < 0;
    unsigned __int128 mag = neg ? (unsigned __int128)(-acc) : (unsigned __int128)acc;
    int msb = 127 - (int)((mag >> 64) ? __builtin_clzll((uint64_t)(mag >> 64)) : 64 + __builtin_clzll((uint64_t)mag));
    int start = msb - 63;
    uint64_t hi64;
    int sticky = 0;
    if (start >= 0) {
      hi64 = (uint64_t)(mag >> start);
      if (start > 0) sticky = (mag & (((unsigned __int128)1 << start) - 1)) != 0;
    } else {
      hi64 = (uint64_t)mag << (-start);
    }
    return round_to_bf16(neg, hi64, start + emin, sticky);
  }
  big_t acc;
  memset(&acc, 0, sizeof(acc));
  for (int i = 0; i < cnt; ++i) big_add_shifted(&acc, (int64_t)ma[i] * mb[i], ee[i] - BIG_LSB);
  return big_round(&acc);
}

/* All-pairs exact dots: out[i*N + j] = bf16(A[i,:] . B[j,:]).  A [M,D], B [N,D]. */
void ko_dot_matrix(const uint16_t *A, const uint16_t *B, uint16_t *out, int64_t M, int64_t N, int64_t D,
                   int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 4)
#endif
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) out[i * N + j] = ko_dot_exact_bf16(A + i * D, B + j * D, D);
}

/* Canonical indexer scores (see header comment).
 * q [B,S,H,D] bf16, k batch b rows at k + b*kbs*D, w [B,S,H] (f32 or bf16), out [B,S,T] f32. */
void ko_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w, int w_bf16, float *out, int64_t B,
                       int64_t S, int64_t H, int64_t D, int64_t T, int64_t kbs, int causal, int64_t start_pos,
                       int ratio, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
#endif
  for (int64_t b = 0; b < B; ++b)
    for (int64_t s = 0; s < S; ++s) {
      const int64_t limit = (start_pos + s + 1) / ratio;
      float *orow = out + (b * S + s) * T;
      const uint16_t *qrow = q + ((b * S + s) * H) * D;
      for (int64_t t = 0; t < T; ++t) {
        if (causal && t >= limit) {
          orow[t] = -INFINITY;
          continue;
        }
        const uint16_t *krow = k + (b * kbs + t) * D;
        float G[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t h = 0; h < H; ++h) {
          uint16_t d = ko_dot_exact_bf16(qrow + h * D, krow, D);
          float df = bf2f(d);
          float r = df > 0.0f ? df : 0.0f;
          int g = (int)((h / 4) % 4);
          if (!w_bf16) {
            float wh = ((const float *)w)[(b * S + s) * H + h];
            G[g] = fmaf(r, wh, G[g]);
          } else {
            float wh = bf2f(((const uint16_t *)w)[(b * S + s) * H + h]);
            float p = bf2f(f2bf_rne(r * wh)); /* r*wh exact in fp32 (8x8-bit significands) */
            G[g] = G[g] + p;
          }
        }
        float sc = (G[0] + G[1]) + (G[2] + G[3]);
        if (w_bf16) sc = bf2f(f2bf_rne(sc));
        orow[t] = sc;
      }
    }
}
