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
// then sorted (descending) on the 64-bit composite (key, ~column), which is exactly (score desc, column
// asc): every wave sorts runs of 128 in registers (bitonic, DPP / permlane exchanges), then merge-path
// rounds through LDS double the runs, one barrier per round.
//
// Causal rows: columns >= limit = (start_pos + s + 1) / ratio are -inf by definition of the masked
// scores (baseline/indexer.py:185-193), so they are never read: the valid prefix is selected and, when
// it holds fewer than k columns, the remaining slots are the masked columns in ascending order, which
// post-processing turns into -1 (the reference's prefix pruning, indexer_topk.asc:96-152).
#include "common.h"
#include "indexer_common.h"
#include "indexer_exact.h"

#include <type_traits>

namespace ks {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkMaxK = 4096;

// score_key (indexer_common.h): key 0 is reserved for "absent" (it would be a negative NaN, which is outside the
// contract).

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

// Inclusive prefix sum over the NW waves of the block (lane order).  `wsum` is NW ints of LDS.
// TRAIL: end with a barrier so that wsum may be rewritten at once; without it the caller must pass a
// barrier before the next scan on the same wsum.
template <bool TRAIL = true, int NW = kTopkWaves>
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v, uint32_t *wsum) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  // the preceding waves' totals: every one read at once (a loop to the wave's index would wait for each read)
  uint32_t base = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t x = wsum[w];
    base += w < wave ? x : 0u;
  }
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

// Outputs [d0, d1) of the merge of two descending lists of unique composites x[0, nx) and y[0, ny)
// (d1 <= nx + ny): the start on the merge path by binary search, then sequential steps.  emit(e, v)
// receives output e.
template <typename Emit>
__device__ __forceinline__ void merge_path(const uint64_t *x, int nx, const uint64_t *y, int ny, int d0, int d1,
                                           Emit emit) {
  // i = how many of the first d0 outputs come from x: the smallest i with x[i] < y[d0 - i - 1]
  int lo = d0 - ny > 0 ? d0 - ny : 0, hi = d0 < nx ? d0 : nx;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (x[mid] > y[d0 - mid - 1]) lo = mid + 1;
    else hi = mid;
  }
  int i = lo, j = d0 - lo;
  for (int e = d0; e < d1; ++e) {
    const bool from_x = j >= ny || (i < nx && x[i] > y[j]);
    emit(e, from_x ? x[i++] : y[j++]);
  }
}

// The first m outputs of that merge over the workgroup: thread t emits outputs [t E, t E + E), E = ceil(m / 1024).
template <typename Emit>
__device__ __forceinline__ void merge_first(const uint64_t *x, int nx, const uint64_t *y, int ny, int m, Emit emit) {
  const int E = (m + kTopkThreads - 1) / kTopkThreads;
  const int d0 = static_cast<int>(threadIdx.x) * E;
  if (d0 < m) merge_path(x, nx, y, ny, d0, d0 + E < m ? d0 + E : m, emit);
}

// Lanes l of register r whose element r*64 + l keeps the larger value in the bitonic stage (SIZE, S): a
// compile-time lane mask.
template <int SIZE, int S, int R>
constexpr uint64_t keep_max_lanes() {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l) {
    const int e = R * 64 + l;
    if (((e & SIZE) == 0) == ((e & S) == 0)) m |= uint64_t(1) << l;
  }
  return m;
}

// Bitonic sort (descending) of a wave's run of 128 composites, element r*64 + lane in v[r]: the exchange at
// distance 64 stays in the lane, the others go through DPP / permlane.  V is uint64_t (key, ~column) or uint32_t
// (a narrower composite of the same order: one lane exchange and one compare per element and stage).  The
// direction of each exchange is a constant lane mask: the compare's lane mask is flipped by it with scalar
// instructions and selects directly (one compare and one select per element and stage).
template <int SIZE, int S, typename V>
__device__ __forceinline__ void run_stage(V (&v)[2], int lane) {
  if constexpr (S == 64) {
    const V a = v[0], c = v[1];  // SIZE == 128: one descending pair
    v[0] = a > c ? a : c;
    v[1] = a > c ? c : a;
  } else {
    V pv[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      if constexpr (sizeof(V) == 8) {
        const uint32_t lo = lane_xor<S>(static_cast<uint32_t>(v[r]));
        const uint32_t hi = lane_xor<S>(static_cast<uint32_t>(v[r] >> 32));
        pv[r] = (static_cast<uint64_t>(hi) << 32) | lo;
      } else {
        pv[r] = lane_xor<S>(v[r]);
      }
    }
    const uint64_t take0 = ~(__builtin_amdgcn_ballot_w64(pv[0] > v[0]) ^ keep_max_lanes<SIZE, S, 0>());
    const uint64_t take1 = ~(__builtin_amdgcn_ballot_w64(pv[1] > v[1]) ^ keep_max_lanes<SIZE, S, 1>());
    v[0] = __builtin_amdgcn_inverse_ballot_w64(take0) ? pv[0] : v[0];
    v[1] = __builtin_amdgcn_inverse_ballot_w64(take1) ? pv[1] : v[1];
  }
  if constexpr (S > 1) run_stage<SIZE, S / 2>(v, lane);
}
template <int SIZE, typename V>
__device__ __forceinline__ void run_sort(V (&v)[2], int lane) {
  run_stage<SIZE, SIZE / 2>(v, lane);
  if constexpr (SIZE < 128) run_sort<SIZE * 2>(v, lane);
}

// Sort (descending) of the composites cand[0, n) (absent = 0 sorts last; P = pow2 >= max(n, 128)) and
// store of the first k_sel in order.  Every wave sorts runs of 128 in registers (run_sort, no barrier);
// log2(P / 128) merge-path rounds then double the runs through the two halves of cand[0, 2P), one
// barrier each, and the last round stores.  ~10 dependent LDS reads per round per thread, against the
// bitonic network's log2(P) (log2(P) + 1) / 2 stages, of which those at distances >= 64 need a barrier.
__device__ void sort_merge_store(uint64_t *cand, int P, int n, int k_sel, int64_t row, int k, void *out,
                                 int out_i64, int causal, int64_t limit, int64_t offset, uint64_t *part) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto emit_final = [&](int e, uint64_t v) {
    if (part != nullptr) {
      part[e] = v;
    } else {
      const int64_t col = static_cast<int64_t>(~static_cast<uint32_t>(v & 0xFFFFFFFFull));
      store_index(out, out_i64, row * k + e, col, causal, limit, offset);
    }
  };
  const int runs = P / 128;
  for (int rr = wave; rr < runs; rr += kTopkWaves) {
    uint64_t v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int e = rr * 128 + r * 64 + lane;
      v[r] = e < n ? cand[e] : 0ull;
    }
    run_sort<2>(v, lane);
    if (runs == 1) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (r * 64 + lane < k_sel) emit_final(r * 64 + lane, v[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 2; ++r) cand[rr * 128 + r * 64 + lane] = v[r];
    }
  }
  if (runs == 1) return;
  __syncthreads();
  uint64_t *src = cand, *dst = cand + P;
  const int E = P > kTopkThreads ? P / kTopkThreads : 1;  // outputs per thread and round
  for (int L = 128; L < P; L <<= 1) {  // every thread runs every round (P is uniform)
    const int d = tid * E;
    const int pair = d / (2 * L), d0 = d % (2 * L);
    const uint64_t *x = src + pair * 2 * L;
    if (2 * L == P) {  // the last round: the first k_sel outputs only
      if (d < k_sel) merge_path(x, L, x + L, L, d0, d0 + (k_sel - d < E ? k_sel - d : E), emit_final);
    } else {
      if (d < P) {
        uint64_t *z = dst + pair * 2 * L;
        merge_path(x, L, x + L, L, d0, d0 + E, [&](int e, uint64_t v) { z[e] = v; });
      }
      __syncthreads();
      uint64_t *t = src;
      src = dst;
      dst = t;
    }
  }
}

// Exact selection of the k_sel largest keys of a row held in registers (column j*1024 + lane), then the
// sorted store.  sh.k_rem == k_sel and sh.hist[0] == 0 on entry, behind a barrier.
template <int KPT>
__device__ __forceinline__ void select_sort_store(const uint32_t (&key)[KPT], int k_sel, int64_t row, int k, void *out, int out_i64,
                                  int causal, int64_t limit, int64_t offset, uint64_t *cand, SelShared &sh,
                                  int col0 = 0, uint64_t *part = nullptr) {
  const int tid = threadIdx.x;
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
      const uint32_t col = static_cast<uint32_t>(col0 + j * kTopkThreads + tid);
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
        const uint32_t col = static_cast<uint32_t>(col0 + j * kTopkThreads + tid);
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

  // ---- sort of the winners (descending composite) and the store
  int P = 128;
  while (P < k_sel) P <<= 1;
  sort_merge_store(cand, P, k_sel, k_sel, row, k, out, out_i64, causal, limit, offset, part);
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

  // every load is issued before the first wait: columns past the valid prefix read column 0 of the row (in
  // bounds: T >= 1) and are masked afterwards, so no load sits behind a branch
  float f[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int col = j * kTopkThreads + tid;
    f[j] = src[col < n_valid ? col : 0];
  }
  uint32_t key[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) key[j] = j * kTopkThreads + tid < n_valid ? score_key(f[j]) : 0u;
  if (tid == 0) sh.k_rem = static_cast<uint32_t>(k_sel);
  for (int i = tid; i < 2048; i += kTopkThreads) sh.hist[0][i] = 0;
  __syncthreads();

  if (k_sel > 0) select_sort_store<KPT>(key, k_sel, row, k, out, out_i64, causal, limit, offset, cand, sh);

  // ---- masked tail: fewer valid columns than k (the -inf ties, in ascending column order)
  for (int j = k_sel + tid; j < k; j += kTopkThreads)
    store_index(out, out_i64, row * k + j, static_cast<int64_t>(n_valid) + (j - k_sel), causal, limit, offset);
}

// ---------------------------------------------------------------- short rows: one wave per row
// Rows of at most 1024 columns with k <= 128 (the drop-in indexer's compressed rows: 650 columns, k = 128):
// a 1024-lane workgroup per row spends its time in barriers, so here every wave owns a row and no barrier
// is used.  Lane l holds columns 64 j + l (j < KPT).  The k-th largest key comes from four 8-bit radix
// passes through the wave's own 256-bin LDS histogram (a wave scan over the bins finds the bucket); keys
// above it are collected with ballots, keys equal to it in column order (j, then lane) up to the count
// needed; the k winners are then sorted as composites (key, ~column) by the in-register bitonic network
// of 128 (two per lane) and stored with the post-processing: the order of topk_rows_kernel.
// The kernel is bound by its VALU work per row, so work that cannot change the result is skipped, by
// wave-uniform branches: column groups j past the row's valid prefix (the causal limit leaves most rows far
// fewer valid columns than T); the whole selection when every valid column is taken; and, when every key's low
// 16 bits follow from its sign (bf16-valued scores, as with bf16 weights), so that a key is fixed by its top 16
// bits, the last two radix passes and half of the sort's work (32-bit composites).
// Rows (waves) per workgroup: small workgroups leave and are replaced independently, so that the waves of a CU are
// spread over the load, selection and sort phases instead of moving through them together (16-row workgroups
// kept every wave of a CU in the same phase: 35.5 -> 30.3 us at the drop-in shape; 2 or 1 rows time the same as 4).
constexpr int kWaveRows = 4;
constexpr int kWaveThreads = kWaveRows * 64;

__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t b) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b), 0u));
}

template <int KPT>
__global__ __launch_bounds__(kWaveThreads) void topk_wave_kernel(const float *__restrict__ scores, int64_t ld,
                                                                int64_t rows, int64_t S, int T, int k, int causal,
                                                                int64_t start_pos, int ratio, int64_t offset,
                                                                void *__restrict__ out, int out_i64, int bf16_vals) {
  __shared__ uint32_t hist[kWaveRows][256];
  __shared__ uint64_t cand[kWaveRows][128];
  // the row index in scalar registers (rows < 2^31, checked by the caller): its remainder by S is a 32-bit scalar
  // division, not a 64-bit vector one
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row32 = blockIdx.x * kWaveRows + static_cast<uint32_t>(wave);
  const int64_t row = row32;
  if (row >= rows) return;  // uniform per wave; the kernel has no barrier
  const int64_t s = row32 % static_cast<uint32_t>(S);
  int64_t limit = INT64_MAX;
  int n_valid = T;
  if (causal) {
    limit = (start_pos + s + 1) / ratio;
    n_valid = static_cast<int>(limit < 0 ? 0 : (limit < T ? limit : T));
  }
  const int k_sel = k < n_valid ? k : n_valid;
  const int jn = (n_valid + 63) / 64;  // column groups holding a valid column (uniform)
  const float *src = scores + row * ld;
  float f[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {  // every load before the first wait (column 0 stands in past the prefix)
    const int col = 64 * j + lane;
    f[j] = src[col < n_valid ? col : 0];
  }
  uint32_t key[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) key[j] = 64 * j + lane < n_valid ? score_key(f[j]) : 0u;
  // every key fixed by its top 16 bits (uniform): checked, unless the caller's scores are bf16 values by
  // construction (bf16_vals: the fused indexer's scores with bf16 weights, rounded to bf16)
  bool top16 = bf16_vals != 0;
  if (!top16) {
    bool odd_low = false;  // a valid key whose low 16 bits do not follow from its sign
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const uint32_t low = key[j] & 0xFFFFu;
      odd_low = odd_low || (key[j] != 0u && low != ((key[j] >> 31) ? 0u : 0xFFFFu));
    }
    top16 = __builtin_amdgcn_ballot_w64(odd_low) == 0ull;
  }
  if (k_sel > 0) {  // uniform
    uint32_t *h = hist[wave];
    uint32_t prefix = 0, mask = 0, k_rem = static_cast<uint32_t>(k_sel), eq_total = 0;
    // every valid key taken: no selection (key 0 marks the columns past the prefix, which no key exceeds)
    const bool take_all = k_sel == n_valid;
    const int npass = take_all ? 0 : (top16 ? 2 : 4);
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      if (pass >= npass) break;
      const int shift = 24 - 8 * pass;
#pragma unroll
      for (int i = 0; i < 4; ++i) h[64 * i + lane] = 0u;
      wave_lds_order();
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        if (j < jn && key[j] != 0u && (key[j] & mask) == prefix) atomicAdd(&h[(key[j] >> shift) & 255u], 1u);
      wave_lds_order();
      // lane l owns bins 255 - 4l .. 252 - 4l: a lane-order inclusive scan is a suffix sum from the top bin
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = h[255 - 4 * lane - i];
      wave_lds_order();  // the next pass clears the bins after these reads
      const uint32_t mine = c[0] + c[1] + c[2] + c[3];
      const uint32_t incl = wave_incl_scan(mine);
      const uint32_t excl = incl - mine;
      const bool here = excl < k_rem && incl >= k_rem;
      uint32_t digit = 0, rem = 0, cnt = 0;
      if (here) {
        uint32_t acc = excl;
        bool found = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (!found && acc + c[i] >= k_rem) {
            digit = static_cast<uint32_t>(255 - 4 * lane - i);
            rem = k_rem - acc;
            cnt = c[i];
            found = true;
          }
          acc += c[i];
        }
      }
      const int src_lane = __builtin_ctzll(__builtin_amdgcn_ballot_w64(here));
      digit = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(digit), src_lane));
      rem = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rem), src_lane));
      cnt = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cnt), src_lane));
      prefix |= digit << shift;
      mask |= 255u << shift;
      k_rem = rem;
      eq_total = cnt;
    }
    // the k_sel-th of the nonzero keys (>= 1); after two passes the low 16 bits follow from the sign bit.  With
    // every key taken, kstar = 0 and take_eq = 0: every nonzero key is above it.
    const uint32_t kstar = take_all ? 0u : (npass == 2 ? (prefix | ((prefix >> 31) ? 0u : 0xFFFFu)) : prefix);
    const uint32_t take_eq = take_all ? 0u : k_rem, n_gt = static_cast<uint32_t>(k_sel) - take_eq;
    (void)eq_total;
    uint64_t *cw = cand[wave];
    uint32_t base_gt = 0, base_eq = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      if (j >= jn) break;
      const bool gt = key[j] > kstar, eq = key[j] == kstar;
      const uint64_t bg = __builtin_amdgcn_ballot_w64(gt), be = __builtin_amdgcn_ballot_w64(eq);
      const uint32_t col = static_cast<uint32_t>(64 * j + lane);
      if (gt) cw[base_gt + lanes_below(bg)] = (static_cast<uint64_t>(key[j]) << 32) | static_cast<uint64_t>(~col);
      const uint32_t re = base_eq + lanes_below(be);
      if (eq && re < take_eq) cw[n_gt + re] = (static_cast<uint64_t>(kstar) << 32) | static_cast<uint64_t>(~col);
      base_gt += static_cast<uint32_t>(__builtin_popcountll(bg));
      base_eq += static_cast<uint32_t>(__builtin_popcountll(be));
    }
    wave_lds_order();
    if (top16) {
      // keys fixed by their top 16 bits, columns below 1024: the 32-bit composite (key bits 31-16,
      // 0xFFFF - column) orders the winners as (key, ~column) does (absent = 0 still sorts last: a valid key's
      // top 16 bits are nonzero)
      uint32_t v[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = r * 64 + lane;
        const uint64_t c = e < k_sel ? cw[e] : 0ull;
        v[r] = (static_cast<uint32_t>(c >> 32) & 0xFFFF0000u) | (static_cast<uint32_t>(c) & 0xFFFFu);
      }
      run_sort<2>(v, lane);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = r * 64 + lane;
        if (e < k_sel) store_index(out, out_i64, row * k + e, 0xFFFF - static_cast<int64_t>(v[r] & 0xFFFFu), causal,
                                   limit, offset);
      }
    } else {
      uint64_t v[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = r * 64 + lane;
        v[r] = e < k_sel ? cw[e] : 0ull;
      }
      run_sort<2>(v, lane);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = r * 64 + lane;
        if (e < k_sel) {
          const int64_t col = static_cast<int64_t>(~static_cast<uint32_t>(v[r] & 0xFFFFFFFFull));
          store_index(out, out_i64, row * k + e, col, causal, limit, offset);
        }
      }
    }
  }
  // ---- masked tail: fewer valid columns than k (the -inf ties, in ascending column order)
  for (int j = k_sel + lane; j < k; j += 64)
    store_index(out, out_i64, row * k + j, static_cast<int64_t>(n_valid) + (j - k_sel), causal, limit, offset);
}

template <int KPT>
int launch_topk_wave(const float *scores, int64_t ld, int64_t rows, int64_t S, int T, int k, int causal,
                     int64_t start_pos, int ratio, int64_t offset, void *out, int out_i64, hipStream_t stream,
                     int bf16_vals) {
  hipLaunchKernelGGL(topk_wave_kernel<KPT>, dim3(static_cast<unsigned>(ceil_div(rows, kWaveRows))),
                     dim3(kWaveThreads), 0, stream, scores, ld, rows, S, T, k, causal, start_pos, ratio, offset, out,
                     out_i64, bf16_vals);
  KS_CHECK_LAUNCH("topk_wave_kernel");
  return KS_OK;
}

template <int KPT>
int launch_topk(const float *scores, int64_t ld, int64_t rows, int64_t S, int T, int k, int causal, int64_t start_pos,
                int ratio, int64_t offset, void *out, int out_i64, hipStream_t stream) {
  int P = 128;  // the sort's runs of 128
  while (P < k) P <<= 1;
  const size_t shmem = static_cast<size_t>(2 * P) * sizeof(uint64_t);  // candidates, then the exchange buffers
  hipLaunchKernelGGL(topk_rows_kernel<KPT>, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), shmem, stream,
                     scores, ld, S, T, k, causal, start_pos, ratio, offset, out, out_i64);
  KS_CHECK_LAUNCH("topk_rows_kernel");
  return KS_OK;
}


// Histogram slices per row: enough workgroups for the 256 CUs, at most kTopkMaxSlices (the recomputation sums
// that many bucket counts per row), at least 1024 columns each.
constexpr int kTopkMaxSlices = 4;
inline int topk_slices(int64_t rows, int T) {
  if (rows >= 256) return 1;
  int p = static_cast<int>((256 + rows - 1) / rows);
  if (p > kTopkMaxSlices) p = kTopkMaxSlices;
  while (p > 1 && T / p < kTopkThreads) --p;
  return p;
}

// Capacity (composites) of a row's list of exact scores >= tau: the power of two >= T up to 8192 (a longer list
// takes the whole-row fallback; k <= 2048 on this path, and the 11-bit threshold bucket can hold ~2000 more).
constexpr int kTopkListCap = 8192;
inline int topk_list_cap(int T) {
  int c = 128;
  while (c < T && c < kTopkListCap) c <<= 1;
  return c;
}

// 64-bit workspace slots of the bounded selection: the rows' lists, their slices' bucket counts (2048 x 32 bits
// each), the rows' states (list length, threshold, largest key: 4 x 32 bits).
inline int64_t topk_bounded_slots(int64_t rows, int NP, int cap) { return rows * cap + rows * NP * 1024 + rows * 2; }

// Wave-wide minimum and maximum (every lane receives both).
__device__ __forceinline__ void wave_min_max(uint32_t &mn, uint32_t &mx) {
#define KS_MM(S)                                             \
  {                                                          \
    const uint32_t a = lane_xor<S>(mn), b = lane_xor<S>(mx); \
    mn = a < mn ? a : mn;                                    \
    mx = b > mx ? b : mx;                                    \
  }
  KS_MM(1) KS_MM(2) KS_MM(4) KS_MM(8) KS_MM(16) KS_MM(32)
#undef KS_MM
}

// ---------------------------------------------------------------- rows of bounded scores
// Bounded scores S with bounds U (the exact score lies in [S - U, S + U]; U = 0 exactly when S is exact) are
// selected in three launches (two where the score kernel has counted the rows, TopkRecompute::counted):
//  1. topk_slice_hist_kernel, workgroup (row, slice): counts of the first 11-bit digit (2048 buckets) of the lower
//     ends S - U of the slice's columns.
//  2. topk_recompute_kernel, workgroup (row, segment): the threshold tau from the row's summed counts (the lower
//     edge of the bucket holding the row's k-th largest lower end, so no exact score of the top k lies below it);
//     every score of the segment with U > 0 whose upper end reaches tau is recomputed exactly and written back
//     (S = exact, U = 0); every column whose upper end reaches tau has a slot in the row's list, which receives
//     the composite (key, ~column) of its exact score, or key 0 (an empty slot) where that score fell below tau.
//  3. topk_collected_kernel, one workgroup per row: the list holds every column of the top k, each with its exact
//     score, so sorting its nonempty slots gives the top k.  A list longer than its capacity falls back to the exact selection over
//     the whole row, whose keys are exact wherever they reach tau (the others enter as upper ends, below tau).
constexpr int kRecD = 128;        // head dim of the recomputation
constexpr int kRecH = 64;         // heads
constexpr int kRecC = kRecD / 8;  // 16-byte chunks per row
constexpr int kRecThreads = 512;  // the recomputation's workgroup
constexpr int kRecWaves = kRecThreads / 64;

// The row's query (64 heads) staged once per workgroup: rows in LDS with a 16-byte XOR swizzle (chunk c of
// head h at c ^ (h & 15): the 16 lanes reading one chunk of 16 heads hit distinct banks), and the head
// weights and statistics.
struct RecShared {
  uint4 q[kRecH * kRecC];
  float w[kRecH];
  float qn[kRecH];
  float qd[kRecH];  // bound_c 2^-23 (qn + 2^-122): the per-head factor of the interval half-widths
  int32_t qsp[kRecH];
};

__device__ __forceinline__ uint4 rec_q(const RecShared &rs, int h, int c) { return rs.q[h * kRecC + (c ^ (h & 15))]; }

// Per-wave scratch of the recomputation: the tile's 16 key rows (row-major, 16-byte XOR swizzle) and the
// tile's near-tie dot list with the exact values.
constexpr int kNearCap = 256;  // near-tie dots listed at a time (a tile has at most 64 x 16)
struct RecWave {
  uint4 k[16 * kRecC];
  int32_t ksp[16];         // the tile's key spans
  uint16_t ent[kNearCap];  // lane << 4 | head bit (4 m + r); overwritten by the dot's exact value
  int64_t limb[18];        // the integer accumulator of the rare dots beyond the double-precision paths
};

// Exact scores of the keys list[0 .. n) of one row, by the canonical contract, written over the row's
// scores (srow, with bound 0 in urow) and over the keys' list slots (bit patterns of the scores).  Each wave takes tiles of 16 keys: four
// 16-head MFMA rounds (heads 16m + 4g + r, m = 0..3) with the score kernel's interval test (same
// half-widths: bound_c 2^-23 ||q_h|| times the key block's norm maximum) keep the relu'd lower ends of all
// 64 heads; the tile's near-tie dots are then recomputed exactly, 16 at a time with a quad of lanes per dot
// (q_h and the key row from LDS: exact_dot_bf16's arithmetic), and the fp32 fma head sum runs in the
// canonical order over the corrected values.  F8: the key rows are e4m3 codes with row scales, dequantised in
// registers to the contract's bf16 rows (q comes dequantised).
template <int NW, bool F8>
__device__ void recompute_scores(int32_t *list, int n, float *srow, float *urow, const TopkRecompute &rc,
                                 const RecShared &rs, RecWave &rw, int64_t kbrow0, int64_t kmax_row0, float qpmax,
                                 uint32_t &n_exact, uint32_t &n_unres) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int ntile = (n + 15) / 16;
  for (int t = wave; t < ntile; t += NW) {
    const int li = 16 * t + l16;
    const bool kv = li < n;
    const int col = list[kv ? li : n - 1];
    const int64_t krow = kbrow0 + col;
    // the tile's loads go out together (one round trip): key rows, key span, key-block norm maximum
    uint4 kb[kRecD / 32];
    uint2 kc8[F8 ? kRecD / 32 : 1];
    float kscale = 0.f;
    if constexpr (F8) {
#pragma unroll
      for (int kk = 0; kk < kRecD / 32; ++kk) kc8[kk] = *reinterpret_cast<const uint2 *>(rc.kc + krow * kRecD + 32 * kk + 8 * g);
      kscale = rc.ks[krow];
    } else {
#pragma unroll
      for (int kk = 0; kk < kRecD / 32; ++kk) kb[kk] = *reinterpret_cast<const uint4 *>(rc.k + krow * kRecD + 32 * kk + 8 * g);
    }
    const int32_t ksv = rc.ksp[krow];
    const float knm = rc.kmax[kmax_row0 + col / kScoreKeyBlock];
    if constexpr (F8) {
      if (__builtin_amdgcn_ballot_w64(!fp8_scale_pow2(kscale)) == 0ull) {
#pragma unroll
        for (int kk = 0; kk < kRecD / 32; ++kk) kb[kk] = fp8_dequant8<true>(kc8[kk], kscale);
      } else {
#pragma unroll
        for (int kk = 0; kk < kRecD / 32; ++kk) kb[kk] = fp8_dequant8<false>(kc8[kk], kscale);
      }
    }
#pragma unroll
    for (int kk = 0; kk < kRecD / 32; ++kk) rw.k[l16 * kRecC + ((4 * kk + g) ^ l16)] = kb[kk];
    rw.ksp[l16] = ksv;  // the four lanes of a key write the same span; read by the near-tie dots below
    uint32_t pl[8];     // relu'd lower ends, heads 16m + 4g + (0, 1) | (2, 3): pl[2m], pl[2m + 1]
    uint32_t ntm = 0;   // bit 4m + r: head 16m + 4g + r is a near tie
    // Interval half-widths: one fma per dot from the per-head factor qd (two roundings, within the three that
    // the bound constant allows for evaluating the width, so the width still bounds the MFMA error; it need not
    // equal the score kernel's, since any valid width certifies the same exact values).  When the query's
    // largest padded norm times a key block's reaches 2^126 (uniform over the wave, and rare), the MFMA may
    // overflow: every dot of the tile is then taken as a near tie and computed exactly.
    const float kp = knm + 0x1p-122f;
    const bool overflow = __builtin_amdgcn_ballot_w64(!(qpmax * kp < 0x1p126f)) != 0ull;
#pragma unroll
    for (int m = 0; m < kRecH / 16; ++m) {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < kRecD / 32; ++kk) acc = mfma16(rec_q(rs, 16 * m + l16, 4 * kk + g), kb[kk], acc);
#pragma unroll
      for (int rp = 0; rp < 2; ++rp) {
        const int h0 = 16 * m + 4 * g + 2 * rp;
        const float d0 = __builtin_fmaf(rs.qd[h0], kp, 0x1p-144f), d1 = __builtin_fmaf(rs.qd[h0 + 1], kp, 0x1p-144f);
        const uint32_t lo = cvt_relu_pk(acc[2 * rp] - d0, acc[2 * rp + 1] - d1);
        const uint32_t hi = cvt_relu_pk(acc[2 * rp] + d0, acc[2 * rp + 1] + d1);
        pl[2 * m + rp] = lo;
        const uint32_t x = lo ^ hi;
        ntm |= ((x & 0xFFFFu) != 0u && kv ? 1u : 0u) << (4 * m + 2 * rp);
        ntm |= ((x >> 16) != 0u && kv ? 1u : 0u) << (4 * m + 2 * rp + 1);
      }
    }
    if (overflow) ntm = kv ? 0xFFFFu : 0u;
    if (__builtin_amdgcn_ballot_w64(ntm != 0u) != 0ull) {
      const uint32_t cnt = __builtin_popcount(ntm);
      const uint32_t incl = wave_incl_scan(cnt);
      const int nd = static_cast<int>(__builtin_amdgcn_readlane(incl, 63));
      const int pos0 = static_cast<int>(incl - cnt);
      const int dq = lane >> 1, sub = lane & 1;  // a pair of lanes per dot, 8 of the 16 chunks each
      for (int s0 = 0; s0 < nd; s0 += kNearCap) {  // list segments of kNearCap dots
        const int ns = nd - s0 < kNearCap ? nd - s0 : kNearCap;
        {
          uint32_t mm = ntm;
          int p = pos0;
          while (mm) {
            const int bit = __builtin_ctz(mm);
            mm &= mm - 1;
            if (p >= s0 && p < s0 + ns) rw.ent[p - s0] = static_cast<uint16_t>((lane << 4) | bit);
            ++p;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int b0 = 0; b0 < ns; b0 += 32) {
          const int e = rw.ent[min(b0 + dq, ns - 1)];
          const int sl = e >> 4, bit = e & 15;
          const int h = 16 * (bit >> 2) + 4 * (sl >> 4) + (bit & 3), kl = sl & 15;
          const int span = rs.qsp[h] + rw.ksp[kl];
          const bool split = span > 52;
          double hi = 0.0, lo = 0.0;
          if (__builtin_amdgcn_ballot_w64(split) == 0ull) {
            // four independent fma chains (every partial sum is exact when the span fits 52 bits)
            double a[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              const uint4 qv = rec_q(rs, h, 8 * sub + c);
              const uint4 kv4 = rw.k[kl * kRecC + ((8 * sub + c) ^ kl)];
              const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
              const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
#pragma unroll
              for (int p = 0; p < 4; ++p) {
                a[p] = __builtin_fma(static_cast<double>(unpack_lo(qw[p])), static_cast<double>(unpack_lo(kw[p])), a[p]);
                a[p] = __builtin_fma(static_cast<double>(unpack_hi(qw[p])), static_cast<double>(unpack_hi(kw[p])), a[p]);
              }
            }
            hi = (a[0] + a[1]) + (a[2] + a[3]);
          } else {
            // wide dynamic range (rare): products above / below 2^(top - 38) accumulate separately
            const int li2 = 16 * t + kl;
            const int64_t kr2 = kbrow0 + list[li2 < n ? li2 : n - 1];
            const double thr = split ? ldexp(1.0, frexp_exp(rs.qn[h]) + frexp_exp(rc.kn[kr2]) - 38) : 0.0;
#pragma unroll 1
            for (int c = 0; c < 8; ++c) {
              const uint4 qv = rec_q(rs, h, 8 * sub + c);
              const uint4 kv4 = rw.k[kl * kRecC + ((8 * sub + c) ^ kl)];
              const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
              const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
#pragma unroll
              for (int p = 0; p < 4; ++p) {
                const double p0 = static_cast<double>(unpack_lo(qw[p])) * static_cast<double>(unpack_lo(kw[p]));
                const double p1 = static_cast<double>(unpack_hi(qw[p])) * static_cast<double>(unpack_hi(kw[p]));
                if (!split || fabs(p0) >= thr) hi += p0; else lo += p0;
                if (!split || fabs(p1) >= thr) hi += p1; else lo += p1;
              }
            }
          }
          hi += dpp_f64<0xB1>(hi);  // the pair's two halves (quad_perm [1, 0, 3, 2])
          lo += dpp_f64<0xB1>(lo);
          uint16_t v;
          if (!split && (hi == 0.0 || (fabs(hi) >= 0x1p-126 && fabs(hi) < 0x1p127))) v = round_to_bf16_fast(hi);
          else v = round2_to_bf16(hi, lo);
          // wider still (rare): the integer accumulator, any range, one dot at a time by the whole wave (its limbs
          // in LDS, so the recomputation's register budget does not carry them)
          uint64_t wide = __builtin_amdgcn_ballot_w64(span > 84 && sub == 0 && b0 + dq < ns);
          while (wide) {  // uniform
            const int wl = __builtin_ctzll(wide);
            wide &= wide - 1;
            const int wh = __builtin_amdgcn_readlane(h, wl), wk = __builtin_amdgcn_readlane(kl, wl);
            const uint16_t r = wave_exact_dot_wide_bf16(
                [&](int j) { return reinterpret_cast<const uint32_t *>(&rs.q[wh * kRecC + ((j >> 2) ^ (wh & 15))])[j & 3]; },
                [&](int j) { return reinterpret_cast<const uint32_t *>(&rw.k[wk * kRecC + ((j >> 2) ^ wk)])[j & 3]; },
                rw.limb);
            if (dq == (wl >> 1)) v = r;  // the pair that owns the dot
            if (lane == wl) ++n_unres;   // counted: dots that needed the integer accumulator
          }
          const uint16_t rv = (v & 0x8000u) ? 0 : v;  // ReLU (also maps -0 to +0)
          // each pair reads only its own entry before this write (the value replaces the entry)
          if (sub == 0 && b0 + dq < ns) rw.ent[b0 + dq] = rv;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint32_t mm = ntm;
        int p = pos0;
        while (mm) {
          const int bit = __builtin_ctz(mm);
          mm &= mm - 1;
          if (p >= s0 && p < s0 + ns) {
            const uint16_t v = rw.ent[p - s0];
            const int m = bit >> 2, r = bit & 3;
            const uint32_t sh = (r & 1) ? 16u : 0u;
            uint32_t &word = pl[2 * m + (r >> 1)];
            word = (word & ~(0xFFFFu << sh)) | (static_cast<uint32_t>(v) << sh);
            ++n_exact;
          }
          ++p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    float G = 0.f;
#pragma unroll
    for (int m = 0; m < kRecH / 16; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t p2 = pl[2 * m + (r >> 1)];
        G = __builtin_fmaf((r & 1) ? unpack_hi(p2) : unpack_lo(p2), rs.w[16 * m + 4 * g + r], G);
      }
    const float tot = combine_groups(G);
    // the score replaces its column in the list too (read back from LDS when the batch is the last one):
    // the tile's lanes read their list slots (and lanes past n read slot n - 1, of this same tile) before
    if (g == 0 && kv) {
      srow[col] = tot;
      urow[col] = 0.f;
      list[li] = __builtin_bit_cast(int32_t, tot);
    }
  }
}

// Workgroup (row, slice): counts of the first 11-bit digit (2048 buckets) of the lower ends (score - U; the score
// itself where U = 0) of slice p's valid columns, stored for the recomputation's threshold.  Workgroup (row, 0)
// also clears the row's list length and key maximum (the recomputation appends to the list after this launch).
template <int KPT>
__global__ __launch_bounds__(kTopkThreads) void topk_slice_hist_kernel(const float *scores, const float *bounds,
                                                                      int64_t ld, int64_t S, int T, int causal,
                                                                      int64_t start_pos, int ratio, int W,
                                                                      uint32_t *__restrict__ hist_out,
                                                                      uint32_t *__restrict__ rstate) {
  __shared__ uint32_t hist[2048];
  const int64_t row = blockIdx.x;
  const int64_t s = row % S;
  const int tid = threadIdx.x;
  int n_valid = T;
  if (causal) {
    const int64_t limit = (start_pos + s + 1) / ratio;
    n_valid = static_cast<int>(limit < 0 ? 0 : (limit < T ? limit : T));
  }
  const int c0 = static_cast<int>(blockIdx.y) * W;
  const int nv = n_valid - c0 <= 0 ? 0 : (n_valid - c0 < W ? n_valid - c0 : W);
  const float *src = scores + row * ld + c0;
  const float *ub = bounds + row * ld + c0;
  float sv[KPT], uv[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {  // every load before the first wait (column 0 stands in past the prefix)
    const int col = j * kTopkThreads + tid;
    sv[j] = src[col < nv ? col : 0];
    uv[j] = ub[col < nv ? col : 0];
  }
  if (blockIdx.y == 0 && tid == 0) {
    rstate[4 * row] = 0u;
    rstate[4 * row + 2] = 0u;
  }
  for (int i = tid; i < 2048; i += kTopkThreads) hist[i] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    if (j * kTopkThreads + tid < nv) {
      const uint32_t kk = score_key(uv[j] > 0.f ? sv[j] - uv[j] : sv[j]);
      if (kk != 0) atomicAdd(&hist[kk >> 21], 1u);
    }
  }
  __syncthreads();
  uint32_t *dst = hist_out + (row * gridDim.y + blockIdx.y) * 2048;
  for (int i = tid; i < 2048; i += kTopkThreads) dst[i] = hist[i];
}

// Workgroup (row, segment) of kRecThreads lanes over columns [c0, c0 + SW) of the row's valid prefix, SW =
// kRecThreads KPB (column c0 + j kRecThreads + tid in slot j of thread tid):
//  - tau: the row's NP bucket counts summed (thread t owns the kBPT buckets below 2048 - kBPT t), a block scan
//    from the top bucket finds the bucket holding the row's k-th largest lower end; tau is its lower edge;
//  - recomputation of the scores with U > 0 whose upper end reaches tau (recompute_scores), written back with
//    U = 0;
//  - the segment's columns whose upper end reaches tau fill a range of the row's list (capacity cap composites)
//    reserved on the row's length counter: the exact key of each, or 0 where the exact score fell below tau; the
//    row state also receives tau and an upper bound of its largest key (the largest upper end).
// Row state (4 x 32 bits per row): list length (slots reserved), tau, largest key bound, unused.
template <int KPB, bool F8>
__global__ __launch_bounds__(kRecThreads, 4) void topk_recompute_kernel(float *scores, int64_t ld, int64_t S, int T,
                                                                    int k, int causal, int64_t start_pos, int ratio,
                                                                    TopkRecompute rc, int segs, int NP,
                                                                    const uint32_t *__restrict__ hists,
                                                                    uint64_t *__restrict__ lists, int cap,
                                                                    uint32_t *__restrict__ rstate) {
  constexpr int SW = kRecThreads * KPB;
  __shared__ RecShared rs;
  __shared__ RecWave rw[kRecWaves];
  __shared__ int32_t list[SW];
  __shared__ uint32_t wsum[kRecWaves];
  __shared__ uint32_t s_tau, s_base;
  // workgroups are dealt to the 8 XCDs round-robin (block id mod 8): the segments of one row are placed on one
  // XCD, so its L2 serves the row's query rows and bucket counts to all of them
  const int64_t nblk = gridDim.x;
  const int64_t lb = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int64_t row = lb / segs;
  const int seg = static_cast<int>(lb % segs);
  const int64_t s = row % S, b = row / S;
  const int tid = threadIdx.x;
  int n_valid = T;
  if (causal) {
    const int64_t limit = (start_pos + s + 1) / ratio;
    n_valid = static_cast<int>(limit < 0 ? 0 : (limit < T ? limit : T));
  }
  const int k_row = k < n_valid ? k : n_valid;
  const int c0 = seg * SW;
  const int nv = n_valid - c0 <= 0 ? 0 : (n_valid - c0 < SW ? n_valid - c0 : SW);
  if (k_row == 0 || nv == 0) return;  // uniform, before any barrier: no valid column here
  float *srow = scores + row * ld;
  float *urow = rc.bounds + row * ld;

  // every load goes out before the first wait: the row's query chunks with its head data, the segment's scores
  // and bounds (column c0 stands in past the valid part), and the row's bucket counts (slice 0 stands in for
  // the slices past NP)
  constexpr int kQPT = kRecH * kRecC / kRecThreads;  // q chunks per thread
  constexpr int kBPT = 2048 / kRecThreads;           // buckets per thread (a multiple of 4)
  static_assert(kQPT * kRecThreads == kRecH * kRecC && kBPT % 4 == 0, "chunks and buckets per thread");
  const int64_t qrow0 = row * kRecH;  // rows of q, w and the q statistics: (b S + s) 64 + head
  uint4 qv[kQPT];
#pragma unroll
  for (int i = 0; i < kQPT; ++i) {
    const int idx = tid + i * kRecThreads, h = idx / kRecC, c = idx % kRecC;
    qv[i] = *reinterpret_cast<const uint4 *>(rc.q + (qrow0 + h) * kRecD + 8 * c);
  }
  const int hh = tid & (kRecH - 1);
  const float wv = rc.w[qrow0 + hh], qnv = rc.qn[qrow0 + hh];
  const int32_t qsv = rc.qsp[qrow0 + hh];
  float sv[KPB], uv[KPB];
#pragma unroll
  for (int j = 0; j < KPB; ++j) {
    const int col = j * kRecThreads + tid;
    sv[j] = srow[c0 + (col < nv ? col : 0)];
    uv[j] = urow[c0 + (col < nv ? col : 0)];
  }
  uint4 hv[kTopkMaxSlices][kBPT / 4];
  const uint32_t *hr = hists + row * NP * 2048 + (2048 - kBPT * (tid + 1));
#pragma unroll
  for (int p = 0; p < kTopkMaxSlices; ++p)
#pragma unroll
    for (int u = 0; u < kBPT / 4; ++u) hv[p][u] = *reinterpret_cast<const uint4 *>(hr + (p < NP ? p : 0) * 2048 + 4 * u);
#pragma unroll
  for (int i = 0; i < kQPT; ++i) {
    const int idx = tid + i * kRecThreads, h = idx / kRecC, c = idx % kRecC;
    rs.q[h * kRecC + (c ^ (h & 15))] = qv[i];
  }
  rs.w[hh] = wv;  // four threads write each head entry, the same values
  rs.qn[hh] = qnv;
  rs.qd[hh] = rc.bound_c * 0x1p-23f * (qnv + 0x1p-122f);
  rs.qsp[hh] = qsv;
  // the query's largest padded head norm (lane h of every wave holds head h): decides per tile whether the
  // one-fma half-widths apply
  float qpmax = qnv + 0x1p-122f;
  qpmax = wave_max_f32(qpmax);
  qpmax = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int32_t, qpmax)));

  // ---- tau: bucket e of the thread's kBPT is 2048 - kBPT (tid + 1) + e (the top one is e = kBPT - 1)
  uint32_t hc[kBPT];
#pragma unroll
  for (int e = 0; e < kBPT; ++e) hc[e] = 0u;
#pragma unroll
  for (int p = 0; p < kTopkMaxSlices; ++p) {
    if (p < NP) {
#pragma unroll
      for (int u = 0; u < kBPT / 4; ++u) {
        hc[4 * u] += hv[p][u].x;
        hc[4 * u + 1] += hv[p][u].y;
        hc[4 * u + 2] += hv[p][u].z;
        hc[4 * u + 3] += hv[p][u].w;
      }
    }
  }
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < kBPT; ++e) mine += hc[e];
  const uint32_t kr = static_cast<uint32_t>(k_row);
  {
    const uint32_t incl = block_inclusive_scan<true, kRecWaves>(mine, wsum);
    const uint32_t excl = incl - mine;
    if (excl < kr && incl >= kr) {  // exactly one thread: the row holds n_valid >= k_row nonzero lower ends
      uint32_t acc = excl, bucket = 0;
      bool found = false;
#pragma unroll
      for (int e = kBPT - 1; e >= 0; --e) {
        acc += hc[e];
        if (!found && acc >= kr) {
          bucket = static_cast<uint32_t>(2048 - kBPT * (tid + 1) + e);
          found = true;
        }
      }
      s_tau = bucket << 21;
    }
  }
  __syncthreads();
  const uint32_t tau = s_tau;
  if (seg == 0 && tid == 0) rstate[4 * row + 1] = tau;

  // ---- the segment's candidates (U > 0, upper end >= tau) and its list slots: every column whose upper end
  // reaches tau (the candidates, and the exact scores >= tau) gets a slot, counted before the recomputation so
  // that one block scan counts both (candidates in the low 16 bits, slots in the high 16: at most SW <= 4096 of
  // each per workgroup) and the reservation is made as soon as a wave's own recomputation ends; a candidate whose
  // exact score falls below tau leaves its slot empty (key 0, which the rank store skips).
  // (few registers stay live across the recomputation: the masks share one word, the bases another, and the
  // largest upper end is taken from hik afterwards)
  uint32_t hik[KPB], masks = 0;  // bit j: column j is a candidate; bit 8 + j: it has a slot
  static_assert(KPB <= 8, "masks of up to 8 columns per thread");
#pragma unroll
  for (int j = 0; j < KPB; ++j) {
    const bool v = j * kRecThreads + tid < nv;
    const uint32_t lo = score_key(uv[j] > 0.f ? sv[j] - uv[j] : sv[j]);
    hik[j] = v ? score_key(uv[j] > 0.f ? sv[j] + uv[j] : sv[j]) : 0u;
    if (v && hik[j] >= tau) masks |= (lo != hik[j] ? 0x101u : 0x100u) << j;
  }
  static_assert(SW < 65536, "candidate and slot counts share a 32-bit scan");
  const uint32_t both = __builtin_popcount(masks & 0xFFu) | (__builtin_popcount(masks >> 8) << 16);
  const uint32_t bexcl = block_inclusive_scan<true, kRecWaves>(both, wsum) - both;  // slots << 16 | candidates
  uint32_t ncand = 0, nres = 0;
#pragma unroll
  for (int w = 0; w < kRecWaves; ++w) {
    ncand += wsum[w] & 0xFFFFu;
    nres += wsum[w] >> 16;
  }
  {
    uint32_t p = bexcl & 0xFFFFu;
#pragma unroll
    for (int j = 0; j < KPB; ++j)
      if ((masks >> j) & 1u) list[p++] = c0 + j * kRecThreads + tid;
  }
  __syncthreads();
  uint32_t n_exact = 0, n_unres = 0;
  if (ncand > 0) {
    const int64_t kbrow0 = b * rc.kbs;
    const int64_t kmax_row0 = b * ((T + kScoreKeyBlock - 1) / kScoreKeyBlock);
    recompute_scores<kRecWaves, F8>(list, static_cast<int>(ncand), srow, urow, rc, rs, rw[tid >> 6], kbrow0, kmax_row0, qpmax,
                                n_exact, n_unres);
  }
  // each wave, its own recomputation done (the atomics wait behind no tile load, and the last wave, which holds
  // the fewest tiles, makes the reservation while the others finish theirs): the row's largest key, bounded by
  // the largest upper end, and the workgroup's slots
  {
    uint32_t umax = 0, unused = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < KPB; ++j) umax = ((masks >> (8 + j)) & 1u) && hik[j] > umax ? hik[j] : umax;
    wave_min_max(unused, umax);
    if ((tid & 63) == 0 && umax != 0u) atomicMax(&rstate[4 * row + 2], umax);
  }
  if (tid == kRecThreads - 1) s_base = nres > 0 ? atomicAdd(&rstate[4 * row], nres) : 0u;
  __syncthreads();  // every recomputed score is in its list slot, and the reservation's base is known
  if (rc.stats != nullptr) {
    if (n_exact) atomicAdd(&rc.stats[0], n_exact);
    if (n_unres) atomicAdd(&rc.stats[1], n_unres);
    if (rc.stats_ext && tid == 0 && ncand) atomicAdd(&rc.stats[2], ncand);
  }

  // ---- the reserved slots: the exact key, or 0 where a recomputed score fell below tau
  const float *listf = reinterpret_cast<const float *>(list);
  uint64_t *dst = lists + row * cap;
  uint32_t pos = s_base + (bexcl >> 16), p = bexcl & 0xFFFFu;
#pragma unroll
  for (int j = 0; j < KPB; ++j) {
    if ((masks >> (8 + j)) & 1u) {
      const bool cj = (masks >> j) & 1u;
      uint32_t key = cj ? score_key(listf[p]) : hik[j];
      p += cj ? 1u : 0u;
      if (key < tau) key = 0u;
      const uint32_t col = static_cast<uint32_t>(c0 + j * kRecThreads + tid);
      if (pos < static_cast<uint32_t>(cap)) dst[pos] = (static_cast<uint64_t>(key) << 32) | static_cast<uint64_t>(~col);
      ++pos;
    }
  }
}

// Sorted store of the k_sel largest of n unique composites, entry j * 1024 + tid in v[j] of thread tid, whose keys
// lie in [kmin, kmax], by ranks from a counting sort: 2048 buckets uniform in the key over [kmin, kmax] (the bucket
// is a monotone function of the key, so a higher bucket holds only larger composites); bucket starts from a block
// scan from the top bucket; every entry is scattered into its bucket's range of tmp, and its rank is its bucket's
// start plus the number of its bucket's entries above it.  Three barriers and O(n) work, against the log2(n)
// dependent merge rounds of a sort.  Returns false, having stored nothing, when a bucket holds more than
// kRankBucketMax entries (keys tied or clustered far beyond a smooth distribution); the caller then sorts.  Uses
// sh.hist (counts, then starts), sh.wsum and tmp[0, n).
constexpr int kRankBuckets = 2048;
constexpr int kRankBucketMax = 256;
template <int PER>
__device__ bool rank_store(const uint64_t (&v)[PER], int n, uint32_t kmin, uint32_t kmax, int k_sel, int64_t row,
                           int k, void *out, int out_i64, int causal, int64_t limit, int64_t offset, uint64_t *tmp,
                           SelShared &sh) {
  static_assert(kRankBuckets == 2 * kTopkThreads, "two buckets per thread");
  const int tid = threadIdx.x;
  uint32_t *cnt = sh.hist[0], *start = sh.hist[1];
  cnt[tid] = 0u;
  cnt[tid + kTopkThreads] = 0u;
  __syncthreads();
  const float scale = static_cast<float>(kRankBuckets) / (static_cast<float>(kmax - kmin) + 1.0f);
  uint32_t bk[PER], pos[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    bk[j] = 0u;
    pos[j] = 0u;
    if (j * kTopkThreads + tid < n && (v[j] >> 32) != 0u) {  // key 0: an empty slot, not ranked
      const uint32_t d = static_cast<uint32_t>(static_cast<float>(static_cast<uint32_t>(v[j] >> 32) - kmin) * scale);
      bk[j] = d < kRankBuckets - 1 ? d : kRankBuckets - 1;
      pos[j] = atomicAdd(&cnt[bk[j]], 1u);  // the entry's place in its bucket (arrival order)
    }
  }
  __syncthreads();
  const int hi = kRankBuckets - 1 - 2 * tid;  // buckets hi and hi - 1, scanned from the top
  const uint32_t c_hi = cnt[hi], c_lo = cnt[hi - 1];
  const uint32_t excl = block_inclusive_scan<false>(c_hi + c_lo, sh.wsum) - (c_hi + c_lo);
  start[hi] = excl;
  start[hi - 1] = excl + c_hi;
  if (__syncthreads_or(c_hi > kRankBucketMax || c_lo > kRankBucketMax)) return false;  // uniform
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (j * kTopkThreads + tid < n && (v[j] >> 32) != 0u) tmp[start[bk[j]] + pos[j]] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (j * kTopkThreads + tid < n && (v[j] >> 32) != 0u) {
      const uint32_t s0 = start[bk[j]], c = cnt[bk[j]];
      uint32_t r = s0, e = 0;
      // four members per step, read together (one LDS round trip per step, not per member)
      for (; e + 4 <= c; e += 4) {
        const uint64_t a0 = tmp[s0 + e], a1 = tmp[s0 + e + 1], a2 = tmp[s0 + e + 2], a3 = tmp[s0 + e + 3];
        r += (a0 > v[j] ? 1u : 0u) + (a1 > v[j] ? 1u : 0u) + (a2 > v[j] ? 1u : 0u) + (a3 > v[j] ? 1u : 0u);
      }
      for (; e < c; ++e) r += tmp[s0 + e] > v[j] ? 1u : 0u;
      if (r < static_cast<uint32_t>(k_sel)) {
        const int64_t col = static_cast<int64_t>(~static_cast<uint32_t>(v[j] & 0xFFFFFFFFull));
        store_index(out, out_i64, row * k + r, col, causal, limit, offset);
      }
    }
  }
  return true;
}

// One workgroup per row: the row's list (every column of its top k, each with its exact score; at least k_sel
// entries) sorted, and the first k_sel stored with the post-processing.  A list past its capacity (its length
// counter still counts every entry) falls back to the exact selection over the row's keys: the score where
// U = 0 (exact, recomputed ones included), the upper end elsewhere (below tau, so below every score of the top k).
template <int KPT>
__global__ __launch_bounds__(kTopkThreads) void topk_collected_kernel(const float *scores, const float *bounds,
                                                                     int64_t ld, int64_t S, int T, int k, int causal,
                                                                     int64_t start_pos, int ratio, int64_t offset,
                                                                     void *__restrict__ out, int out_i64,
                                                                     const uint64_t *__restrict__ lists, int cap,
                                                                     int spec, const uint32_t *__restrict__ rstate) {
  extern __shared__ uint64_t cand[];  // 2 cap composites: the list, then the sort's exchange buffers
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
  if (k_sel > 0) {
    // the length and the list's first spec entries go out together (a list rarely runs much past k; the loads
    // past the length are discarded), the rest of the list once the length asks for it
    const uint4 st = *reinterpret_cast<const uint4 *>(rstate + 4 * row);  // length, tau, largest key
    const uint32_t n = st.x;
    const uint64_t *src = lists + row * cap;
    constexpr int kMaxPer = kTopkListCap / kTopkThreads;
    uint64_t v[kMaxPer];
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
      const int i = j * kTopkThreads + tid;
      v[j] = 0;
      if (j * kTopkThreads < spec) v[j] = src[i < cap ? i : 0];  // uniform
    }
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
      const int i = j * kTopkThreads + tid;
      if (j * kTopkThreads >= spec && j * kTopkThreads < static_cast<int>(n < static_cast<uint32_t>(cap) ? n : cap))
        v[j] = src[i < cap ? i : 0];  // uniform
    }
    if (n >= static_cast<uint32_t>(k_sel) && n <= static_cast<uint32_t>(cap)) {  // uniform
      if (!rank_store<kMaxPer>(v, static_cast<int>(n), st.y, st.z, k_sel, row, k, out, out_i64, causal, limit, offset,
                               cand, sh)) {
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
          const uint32_t i = static_cast<uint32_t>(j * kTopkThreads + tid);
          if (i < n) cand[i] = v[j];
        }
        __syncthreads();
        int P = 128;
        while (P < static_cast<int>(n)) P <<= 1;
        sort_merge_store(cand, P, static_cast<int>(n), k_sel, row, k, out, out_i64, causal, limit, offset, nullptr);
      }
    } else {
      const float *src = scores + row * ld;
      const float *ub = bounds + row * ld;
      float sv[KPT], uv[KPT];
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int col = j * kTopkThreads + tid;
        sv[j] = src[col < n_valid ? col : 0];
        uv[j] = ub[col < n_valid ? col : 0];
      }
      uint32_t key[KPT];
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        key[j] = j * kTopkThreads + tid < n_valid ? score_key(uv[j] > 0.f ? sv[j] + uv[j] : sv[j]) : 0u;
      if (tid == 0) sh.k_rem = static_cast<uint32_t>(k_sel);
      for (int i = tid; i < 2048; i += kTopkThreads) sh.hist[0][i] = 0;
      __syncthreads();
      select_sort_store<KPT>(key, k_sel, row, k, out, out_i64, causal, limit, offset, cand, sh);
    }
  }
  // ---- masked tail: fewer valid columns than k (the -inf ties, in ascending column order)
  for (int j = k_sel + tid; j < k; j += kTopkThreads)
    store_index(out, out_i64, row * k + j, static_cast<int64_t>(n_valid) + (j - k_sel), causal, limit, offset);
}

}  // namespace
}  // namespace ks

// bf16_vals: every score is a bf16 value (the caller's guarantee; the wave form then skips its check of the keys'
// low halves)
int ks::indexer_topk_impl(const float *scores, int64_t ld, int64_t B, int64_t S, int64_t T, int64_t k, int32_t causal,
                          int64_t start_pos, int32_t ratio, int64_t offset, void *out, int32_t out_i64, void *stream,
                          int bf16_vals) {
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
  if (T <= 1024 && k <= 128) {  // short rows: one wave per row
    if (T <= 64) return ks::launch_topk_wave<1>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
    if (T <= 128) return ks::launch_topk_wave<2>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
    if (T <= 256) return ks::launch_topk_wave<4>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
    if (T <= 512) return ks::launch_topk_wave<8>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
    if (T <= 768) return ks::launch_topk_wave<12>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
    return ks::launch_topk_wave<16>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st, bf16_vals);
  }
  if (T <= 1024) return ks::launch_topk<1>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 2048) return ks::launch_topk<2>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 4096) return ks::launch_topk<4>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 8192) return ks::launch_topk<8>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 16384) return ks::launch_topk<16>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  if (T <= 32768) return ks::launch_topk<32>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
  return ks::launch_topk<64>(scores, ld, rows, S, Ti, ki, c, start_pos, ratio, offset, out, o, st);
}

extern "C" int ks_indexer_topk(const float *scores, int64_t ld, int64_t B, int64_t S, int64_t T, int64_t k,
                               int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset, void *out,
                               int32_t out_i64, void *stream) {
  ks::last_error().clear();
  return ks::indexer_topk_impl(scores, ld, B, S, T, k, causal, start_pos, ratio, offset, out, out_i64, stream, 0);
}

int ks::launch_indexer_topk_bounded(float *scores, int64_t ld, int64_t B, int64_t S, int64_t T, int64_t k,
                                    int causal, int64_t start_pos, int ratio, int64_t offset, void *out, int out_i64,
                                    const TopkRecompute &rc, hipStream_t st) {
  KS_CHECK_ARG(B >= 0 && S >= 0 && T >= 1 && T <= 32768 && k >= 1 && k <= T && k <= 2048 && ld >= T && ratio >= 1 &&
                   start_pos >= 0,
               "indexer top-k (bounded): bad arguments");
  const int64_t rows = B * S;
  if (rows == 0) return KS_OK;
  const int Ti = static_cast<int>(T), ki = static_cast<int>(k);
  const int c = causal ? 1 : 0, o = out_i64 ? 1 : 0;
  // counted: the score kernel has counted each row whole (one slice); otherwise the histogram launch counts slices
  const int np = rc.counted ? 1 : topk_slices(rows, Ti);
  int W = kTopkThreads;  // columns per histogram slice: 1024 times a power of two
  while (W * np < Ti) W <<= 1;
  const int NP = (Ti + W - 1) / W;
  const int cap = topk_list_cap(Ti);
  // columns per recomputation thread: 8, 4 or 2, the largest that still gives ~512 workgroups (two per CU; each
  // wave should own about one tile of candidates: the tile's chain of dependent steps, not the arithmetic, sets
  // its time, while every workgroup stages the row's query once)
  int kpb = 8;
  while (kpb > 2 && rows * ((Ti + kRecThreads * kpb - 1) / (kRecThreads * kpb)) < 512) kpb >>= 1;
  const int segs = (Ti + kRecThreads * kpb - 1) / (kRecThreads * kpb);
  KS_CHECK_ARG(rows * segs < (int64_t(1) << 31), "indexer top-k (bounded): too many rows");
  const int64_t need = topk_bounded_slots(rows, NP, cap);
  KS_CHECK_ARG(rc.part != nullptr && rc.part_cap >= need,
               "indexer top-k (bounded): %lld 64-bit workspace slots required, %lld given", (long long)need,
               (long long)rc.part_cap);
  uint64_t *lists = rc.part;
  uint32_t *hists = reinterpret_cast<uint32_t *>(rc.part + rows * cap);
  uint32_t *rstate = hists + rows * NP * 2048;
  const float *bnd = rc.bounds;
  if (!rc.counted) {
    const dim3 hgrid(static_cast<unsigned>(rows), static_cast<unsigned>(NP));
#define KS_HIST(KPT_)                                                                                          \
  hipLaunchKernelGGL(topk_slice_hist_kernel<KPT_>, hgrid, dim3(kTopkThreads), 0, st, scores, bnd, ld, S, Ti, c, \
                     start_pos, ratio, W, hists, rstate)
    switch (W / kTopkThreads) {
      case 1: KS_HIST(1); break;
      case 2: KS_HIST(2); break;
      case 4: KS_HIST(4); break;
      case 8: KS_HIST(8); break;
      case 16: KS_HIST(16); break;
      default: KS_HIST(32); break;
    }
#undef KS_HIST
    KS_CHECK_LAUNCH("topk_slice_hist_kernel");
  }
  const dim3 rgrid(static_cast<unsigned>(rows * segs));
  const bool f8 = rc.kc != nullptr;
  KS_CHECK_ARG(f8 == (rc.ks != nullptr), "indexer top-k (bounded): FP8 keys need codes and scales");
#define KS_REC(KPB_, F8_)                                                                                           \
  hipLaunchKernelGGL((topk_recompute_kernel<KPB_, F8_>), rgrid, dim3(kRecThreads), 0, st, scores, ld, S, Ti, ki, c, \
                     start_pos, ratio, rc, segs, NP, hists, lists, cap, rstate)
  if (f8) {
    if (kpb == 2) KS_REC(2, true);
    else if (kpb == 4) KS_REC(4, true);
    else KS_REC(8, true);
  } else {
    if (kpb == 2) KS_REC(2, false);
    else if (kpb == 4) KS_REC(4, false);
    else KS_REC(8, false);
  }
#undef KS_REC
  KS_CHECK_LAUNCH("topk_recompute_kernel");
  const size_t shmem = static_cast<size_t>(2 * cap) * sizeof(uint64_t);
  // list entries loaded with the length (a multiple of the workgroup): ~1.25 k, which the lists rarely exceed
  const int spec = static_cast<int>(ceil_div(ki + ki / 4, kTopkThreads) * kTopkThreads);
#define KS_COLL(KPT_)                                                                                                \
  hipLaunchKernelGGL(topk_collected_kernel<KPT_>, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), shmem, st, \
                     scores, bnd, ld, S, Ti, ki, c, start_pos, ratio, offset, out, o, lists, cap, spec, rstate)
  if (Ti <= 1024) KS_COLL(1);
  else if (Ti <= 2048) KS_COLL(2);
  else if (Ti <= 4096) KS_COLL(4);
  else if (Ti <= 8192) KS_COLL(8);
  else if (Ti <= 16384) KS_COLL(16);
  else KS_COLL(32);
#undef KS_COLL
  KS_CHECK_LAUNCH("topk_collected_kernel");
  return KS_OK;
}

uint32_t *ks::topk_bounded_counts(uint64_t *part, int64_t rows, int64_t T) {
  // the lists first (rows x cap composites), then one slice of counts per row and the row states, as the
  // launcher lays them out for NP = 1
  return reinterpret_cast<uint32_t *>(part + rows * topk_list_cap(static_cast<int>(T)));
}

int64_t ks::topk_bounded_part_capacity(int64_t rows, int64_t T) {
  if (rows <= 0 || T < 1 || T > 32768) return 0;
  const int Ti = static_cast<int>(T);
  const int np = topk_slices(rows, Ti);
  int W = kTopkThreads;
  while (W * np < Ti) W <<= 1;
  return topk_bounded_slots(rows, (Ti + W - 1) / W, topk_list_cap(Ti));
}

// Diagnostic entry (not part of the public header) of the bounded top-k, for timing it alone: scores and
// bounds from ks_dbg_indexer_scores_bounded over rotated q / k (with their row statistics); the scores that
// are recomputed are rewritten in place (bound 0).  ratio 1, int32 output.  part: part_cap 64-bit slots, at
// least ks_dbg_topk_bounded_slots(B S, T) of them, holding, where the fused entry counts the rows in the score
// kernel (ks::scores_count_rows), the counts that ks_dbg_indexer_scores_bounded accumulated into its zeroed
// count region; otherwise the selection counts the rows itself (its histogram launch).
extern "C" int ks_dbg_indexer_topk_bounded(float *scores, float *bounds, const float *kmax, const uint16_t *q,
                                           const uint16_t *k, const float *w, const float *q_norm,
                                           const int32_t *q_span, const float *k_norm, const int32_t *k_span,
                                           int64_t B, int64_t S, int64_t T, int64_t k_top, int32_t causal,
                                           int64_t start_pos, void *out, void *stream, uint64_t *part,
                                           int64_t part_cap) {
  ks::last_error().clear();
  KS_CHECK_ARG(scores && bounds && kmax && q && k && w && q_norm && q_span && k_norm && k_span && out && part,
               "ks_dbg_indexer_topk_bounded: null pointer");
  KS_CHECK_ARG(T <= 32768 && k_top <= 2048, "ks_dbg_indexer_topk_bounded: T <= 32768 and k <= 2048");
  const ks::TopkRecompute rc{bounds, kmax, q, k, w, q_norm, q_span, k_norm, k_span, T, ks::kScoreBoundC, nullptr, 0,
                             part, part_cap, ks::scores_count_rows(B, S, T) ? 1 : 0};
  return ks::launch_indexer_topk_bounded(scores, T, B, S, T, k_top, causal ? 1 : 0, start_pos, 1, 0, out, 0, rc,
                                         static_cast<hipStream_t>(stream));
}

extern "C" int64_t ks_dbg_topk_bounded_slots(int64_t rows, int64_t T) { return ks::topk_bounded_part_capacity(rows, T); }
