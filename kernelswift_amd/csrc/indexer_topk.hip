// Exact sorted top-k per score row with the reference's -1 / +offset post-processing (gfx950).
//
// Semantics: index_score.topk(k) + post-processing (baseline/indexer.py:195-206), with the tie order
// of a stable descending sort (equal scores keep ascending column order; -inf sorts last) that the
// reference TopK kernel reproduces (optimized/indexer_project/design.md:99-105,
// optimized/indexer_project/op_kernel/indexer_topk.asc:219-246).
//
// One 1024-lane workgroup per row.  The row is read once into registers (column j*1024 + lane),
// converted to order-preserving uint32 keys.  A 3-pass LDS radix select (11 + 11 + 10 bits) finds the
// k-th largest key K*; keys > K* are collected unordered (slots from a block scan), keys == K* are collected
// in column order (ordered block scan) only when more of them exist than are needed.  The k winners are
// then bitonic-sorted (descending) on the 64-bit composite (key, ~column), which is exactly (score desc,
// column asc); the elements stay in registers, and only exchange distances between 64 and the number of
// active threads go through LDS, so the network costs one barrier per such stage instead of per stage.
//
// Causal rows: columns >= limit = (start_pos + s + 1) / ratio are -inf by definition of the masked
// scores (baseline/indexer.py:185-193), so they are never read: the valid prefix is selected and, when
// it holds fewer than k columns, the remaining slots are the masked columns in ascending order, which
// post-processing turns into -1 (the reference's prefix pruning, indexer_topk.asc:96-152).
#include "common.h"

namespace ks {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkMaxK = 4096;

// fp32 -> uint32 whose unsigned order equals the float order; -0 is canonicalised to +0.
// Key 0 is reserved for "absent" (it would be a negative NaN, which is outside the contract).
__device__ __forceinline__ uint32_t score_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP: row shifts by 1, 2, 4, 8 within each 16-lane
// row, then the last lane of row 0 / row 2 broadcast into rows 1 / 3 and lane 31 into rows 2-3.  Lanes
// whose DPP source is outside the row (or whose row is masked off) add 0.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Inclusive prefix sum over the 1024 lanes of the block (lane order).  `wsum` is kTopkWaves ints of LDS.
// TRAIL: end with a barrier so that wsum may be rewritten at once; without it the caller must pass a
// barrier before the next scan on the same wsum.
template <bool TRAIL = true>
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v, uint32_t *wsum) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  uint32_t base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  if constexpr (TRAIL) __syncthreads();
  return v + base;
}

struct SelShared {
  uint32_t hist[2][2048];  // pass p counts into hist[p & 1] while hist[(p + 1) & 1] is cleared
  uint32_t wsum[kTopkWaves];
  uint32_t digit;
  uint32_t k_rem;
  uint32_t bucket_count;
};

// One radix pass: histogram of digit (key >> shift) & (nbins-1) among keys whose bits above the
// digit equal `prefix` under `mask`; then locate the bucket holding the k_rem-th largest.  hist[buf] is
// zero on entry (cleared before the barrier that precedes the pass); hist[buf ^ 1] is cleared here for the
// next pass (its last readers finished before that same barrier).
template <int KPT>
__device__ __forceinline__ void radix_pass(const uint32_t (&key)[KPT], uint32_t prefix, uint32_t mask, int shift,
                                           int nbins, SelShared &sh, int buf) {
  // k_rem must be read before the barrier that precedes this pass's single update of it
  const uint32_t k_rem = sh.k_rem;
  uint32_t *hist = sh.hist[buf];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const uint32_t kk = key[j];
    if (kk != 0 && (kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & (nbins - 1)], 1u);
  }
  for (int i = threadIdx.x; i < 2048; i += kTopkThreads) sh.hist[buf ^ 1][i] = 0;
  __syncthreads();
  // Lane t owns bins hi = nbins-1-2t and lo = hi-1 (two bins per lane for 2048, one for 1024):
  // an inclusive lane-order scan is then a suffix sum over bins from the top.
  const int per = nbins / kTopkThreads;  // 2 or 1
  const int hi = nbins - 1 - per * static_cast<int>(threadIdx.x);
  const uint32_t c_hi = hist[hi];
  const uint32_t c_lo = per == 2 ? hist[hi - 1] : 0u;
  const uint32_t mine = c_hi + c_lo;
  const uint32_t incl = block_inclusive_scan<false>(mine, sh.wsum);  // the barrier below ends the pass
  const uint32_t excl = incl - mine;
  if (excl < k_rem && incl >= k_rem) {
    if (excl + c_hi >= k_rem) {
      sh.digit = static_cast<uint32_t>(hi);
      sh.bucket_count = c_hi;
      sh.k_rem = k_rem - excl;
    } else {
      sh.digit = static_cast<uint32_t>(hi - 1);
      sh.bucket_count = c_lo;
      sh.k_rem = k_rem - excl - c_hi;
    }
  }
  __syncthreads();
}

// Post-processing of one selected column (baseline/indexer.py:198-206) and its store.
__device__ __forceinline__ void store_index(void *out, int out_i64, int64_t at, int64_t col, int causal, int64_t limit,
                                            int64_t offset) {
  const int64_t v = (causal && col >= limit) ? int64_t(-1) : col + offset;
  if (out_i64) {
    static_cast<int64_t *>(out)[at] = v;
  } else {
    static_cast<int32_t *>(out)[at] = static_cast<int32_t>(v);
  }
}

// One bitonic compare-exchange stage at distance S < 64: the partner (lane ^ S) is in the same wave and
// its value arrives through DPP / permlane (no LDS).  A lane keeps the larger composite when it holds the
// lower position of a descending pair or the upper position of an ascending one, so it takes the partner's
// value exactly when (partner > own) == keep_max (on equality either value is the same).
template <int E, int S>
__device__ __forceinline__ void wave_stage(uint64_t (&v)[E], int NT, int size) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int e = r * NT + tid;
    const uint32_t lo = lane_xor<S>(static_cast<uint32_t>(v[r]));
    const uint32_t hi = lane_xor<S>(static_cast<uint32_t>(v[r] >> 32));
    const uint64_t pv = (static_cast<uint64_t>(hi) << 32) | lo;
    const bool keep_max = ((e & size) == 0) == ((e & S) == 0);
    v[r] = ((pv > v[r]) == keep_max) ? pv : v[r];
  }
}

// Bitonic sort (descending) of the P composites cand[0..k_sel) (absent = 0 sorts last) and store of the
// first k_sel in order.  Element e = r*NT + tid lives in registers; compare-exchange partners at distance
// >= NT are in the same thread, at distance < 64 in the same wave (DPP / permlane, the six stages of a
// merge step unrolled at compile time); only distances in between go through LDS (cand[0..2P) as two
// alternating exchange buffers: one barrier per such stage).  Waves holding no elements only join the
// barriers.
template <int E>
__device__ void sort_and_store(uint64_t *cand, int P, int k_sel, int64_t row, int k, void *out, int out_i64,
                               int causal, int64_t limit, int64_t offset) {
  const int tid = threadIdx.x;
  const int NT = P / E < 64 ? 64 : P / E;  // active threads (at least one wave)
  const bool act = tid < NT;               // uniform per wave (NT is a multiple of 64)
  uint64_t v[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int e = r * NT + tid;
    v[r] = (act && e < k_sel) ? cand[e] : 0ull;
  }
  __syncthreads();  // the candidates are in registers; LDS becomes the exchange area
  int phase = 0;
  for (int size = 2; size <= P; size <<= 1) {
    int stride = size >> 1;
    for (; stride >= NT; stride >>= 1) {  // partner in this thread (E > 1)
      if (act) {
        const int rs = stride / NT;
#pragma unroll
        for (int r = 0; r < E; ++r) {
          if ((r & rs) == 0) {
            const int e = r * NT + tid;
            const uint64_t a = v[r], c = v[r | rs];
            const uint64_t hi = a > c ? a : c, lo = a > c ? c : a;
            const bool desc = (e & size) == 0;
            v[r] = desc ? hi : lo;
            v[r | rs] = desc ? lo : hi;
          }
        }
      }
    }
    for (; stride >= 64; stride >>= 1) {  // partner in another wave
      uint64_t *xb = cand + (phase & 1) * P;
      ++phase;
      if (act) {
#pragma unroll
        for (int r = 0; r < E; ++r) xb[r * NT + tid] = v[r];
      }
      __syncthreads();
      if (act) {
#pragma unroll
        for (int r = 0; r < E; ++r) {
          const int e = r * NT + tid;
          const uint64_t pv = xb[e ^ stride];
          const bool keep_max = ((e & size) == 0) == ((e & stride) == 0);
          v[r] = ((pv > v[r]) == keep_max) ? pv : v[r];
        }
      }
    }
    if (act) {  // partner in this wave: strides min(size / 2, 32) .. 1
      if (size >= 64) wave_stage<E, 32>(v, NT, size);
      if (size >= 32) wave_stage<E, 16>(v, NT, size);
      if (size >= 16) wave_stage<E, 8>(v, NT, size);
      if (size >= 8) wave_stage<E, 4>(v, NT, size);
      if (size >= 4) wave_stage<E, 2>(v, NT, size);
      wave_stage<E, 1>(v, NT, size);
    }
  }
  if (act) {
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const int e = r * NT + tid;
      if (e < k_sel) {
        const int64_t col = static_cast<int64_t>(~static_cast<uint32_t>(v[r] & 0xFFFFFFFFull));
        store_index(out, out_i64, row * k + e, col, causal, limit, offset);
      }
    }
  }
}

template <int KPT>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(const float *__restrict__ scores, int64_t ld,
                                                                int64_t S, int T, int k, int causal,
                                                                int64_t start_pos, int ratio, int64_t offset,
                                                                void *__restrict__ out, int out_i64) {
  extern __shared__ uint64_t cand[];  // 2P composites: candidates, then the sort's exchange buffers
  __shared__ SelShared sh;
  const int64_t row = blockIdx.x;
  const int64_t s = row % S;
  const int tid = threadIdx.x;
  int64_t limit = INT64_MAX;
  int n_valid = T;
  if (causal) {
    limit = (start_pos + s + 1) / ratio;
    n_valid = static_cast<int>(limit < 0 ? 0 : (limit < T ? limit : T));
  }
  const int k_sel = k < n_valid ? k : n_valid;
  const float *src = scores + row * ld;

  uint32_t key[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int col = j * kTopkThreads + tid;
    key[j] = col < n_valid ? score_key(src[col]) : 0u;
  }
  if (tid == 0) sh.k_rem = static_cast<uint32_t>(k_sel);
  for (int i = tid; i < 2048; i += kTopkThreads) sh.hist[0][i] = 0;
  __syncthreads();

  if (k_sel > 0) {
    // ---- radix select of the k_sel-th largest key
    radix_pass<KPT>(key, 0u, 0u, 21, 2048, sh, 0);
    const uint32_t d1 = sh.digit;
    radix_pass<KPT>(key, d1 << 21, 0xFFE00000u, 10, 2048, sh, 1);
    const uint32_t d2 = sh.digit;
    radix_pass<KPT>(key, (d1 << 21) | (d2 << 10), 0xFFFFFC00u, 0, 1024, sh, 0);
    const uint32_t kstar = (d1 << 21) | (d2 << 10) | sh.digit;
    const uint32_t take_eq = sh.k_rem;          // how many keys == K* are selected (>= 1)
    const uint32_t eq_total = sh.bucket_count;  // how many keys == K* exist
    const uint32_t n_gt = static_cast<uint32_t>(k_sel) - take_eq;

    // ---- collect keys > K* (unordered) and, if all of them are taken, keys == K*: slots from a block scan
    uint32_t ntake = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) ntake += (key[j] > kstar || (key[j] == kstar && take_eq == eq_total)) ? 1u : 0u;
    uint32_t pos = block_inclusive_scan(ntake, sh.wsum) - ntake;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const uint32_t kk = key[j];
      if (kk > kstar || (kk == kstar && take_eq == eq_total)) {
        const uint32_t col = static_cast<uint32_t>(j * kTopkThreads + tid);
        cand[pos++] = (static_cast<uint64_t>(kk) << 32) | static_cast<uint64_t>(~col);
      }
    }
    // ---- ties at K*: the take_eq lowest columns, found with an ordered scan (column = j*1024 + lane)
    if (take_eq != eq_total) {
      uint32_t base = 0;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const uint32_t f = key[j] == kstar ? 1u : 0u;
        const uint32_t incl = block_inclusive_scan(f, sh.wsum);
        const uint32_t rank = base + incl - f;
        if (f && rank < take_eq) {
          const uint32_t col = static_cast<uint32_t>(j * kTopkThreads + tid);
          cand[n_gt + rank] = (static_cast<uint64_t>(kstar) << 32) | static_cast<uint64_t>(~col);
        }
        // block total of this slice = sum of the per-wave totals left in wsum by the scan
        uint32_t tot = 0;
        for (int w = 0; w < kTopkWaves; ++w) tot += sh.wsum[w];
        base += tot;
        __syncthreads();  // wsum is rewritten by the next slice's scan
      }
    }
    __syncthreads();

    // ---- bitonic sort of the winners (descending composite), P = pow2 >= k_sel elements, E per thread
    int P = 2;
    while (P < k_sel) P <<= 1;
    if (P <= kTopkThreads) {
      sort_and_store<1>(cand, P, k_sel, row, k, out, out_i64, causal, limit, offset);
    } else if (P == 2 * kTopkThreads) {
      sort_and_store<2>(cand, P, k_sel, row, k, out, out_i64, causal, limit, offset);
    } else {
      sort_and_store<4>(cand, P, k_sel, row, k, out, out_i64, causal, limit, offset);
    }
  }

  // ---- masked tail: fewer valid columns than k (the -inf ties, in ascending column order)
  for (int j = k_sel + tid; j < k; j += kTopkThreads)
    store_index(out, out_i64, row * k + j, static_cast<int64_t>(n_valid) + (j - k_sel), causal, limit, offset);
}

template <int KPT>
int launch_topk(const float *scores, int64_t ld, int64_t rows, int64_t S, int T, int k, int causal, int64_t start_pos,
                int ratio, int64_t offset, void *out, int out_i64, hipStream_t stream) {
  int P = 2;
  while (P < k) P <<= 1;
  const size_t shmem = static_cast<size_t>(2 * P) * sizeof(uint64_t);  // candidates, then the exchange buffers
  hipLaunchKernelGGL(topk_rows_kernel<KPT>, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), shmem, stream,
                     scores, ld, S, T, k, causal, start_pos, ratio, offset, out, out_i64);
  KS_CHECK_LAUNCH("topk_rows_kernel");
  return KS_OK;
}

}  // namespace
}  // namespace ks

extern "C" int ks_indexer_topk(const float *scores, int64_t ld, int64_t B, int64_t S, int64_t T, int64_t k,
                               int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset, void *out,
                               int32_t out_i64, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(B >= 0 && S >= 0, "ks_indexer_topk: negative B or S");
  KS_CHECK_ARG(T >= 1 && T <= 65536, "ks_indexer_topk: T=%lld must be in [1, 65536]", (long long)T);
  KS_CHECK_ARG(k >= 1 && k <= T && k <= ks::kTopkMaxK, "ks_indexer_topk: k=%lld must be in [1, min(T, %d)]",
               (long long)k, ks::kTopkMaxK);
  KS_CHECK_ARG(ld >= T, "ks_indexer_topk: ld=%lld < T=%lld", (long long)ld, (long long)T);
  KS_CHECK_ARG(ratio >= 1, "ks_indexer_topk: ratio=%d must be >= 1", ratio);
  KS_CHECK_ARG(start_pos >= 0, "ks_indexer_topk: start_pos must be >= 0");
  const int64_t rows = B * S;
  if (rows == 0) return KS_OK;
  KS_CHECK_ARG(rows < (int64_t(1) << 31), "ks_indexer_topk: too many rows");
  KS_CHECK_ARG(scores != nullptr && out != nullptr, "ks_indexer_topk: null pointer");
  KS_CHECK_ARG(ks::aligned(scores, 4) && ks::aligned(out, out_i64 ? 8 : 4), "ks_indexer_topk: misaligned pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Ti = static_cast<int>(T), ki = static_cast<int>(k);
  const int c = causal ? 1 : 0, o = out_i64 ? 1 : 0;
  if (T <= 1024) return ks::launch_topk<1>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 2048) return ks::launch_topk<2>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 4096) return ks::launch_topk<4>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 8192) return ks::launch_topk<8>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 16384) return ks::launch_topk<16>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 32768) return ks::launch_topk<32>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  return ks::launch_topk<64>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
}
