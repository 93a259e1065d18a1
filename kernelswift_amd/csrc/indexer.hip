// Fused indexer entries: RoPE (or FP8 dequantisation) + row statistics of q and k (one launch) -> scores ->
// exact top-k.
//
// Semantics of baseline/indexer.py:161-206 after the two projections (which stay in the caller):
// RoPE on the configured segment of q (and k), score = sum_h w_h * relu(bf16(q_h . k)), causal mask,
// sorted top-k with lowest-index ties, -1 / +offset post-processing.  Replaces the reference's three-op
// sequence rope_inplace -> fused_qk_reduce -> topk_mask (optimized/indexer_project/indexer.py:197-222).
// All intermediates live in the caller's workspace; inputs are never modified.  RoPE stays a pass of its
// own: done inside the score kernel it would be repeated by every workgroup that reads a row (S/8 times
// per key row), which measured twice as slow as the separate pass.
//
// With 64 heads, D = 128 and fp32 weights the scores are computed with bounds instead of exactly: the
// score kernel keeps the canonical score of the lower interval ends plus a per-score bound, and the top-k
// kernel recomputes exactly only the scores whose interval reaches its selection threshold.  The selected
// indices are identical to those of the exact path (same intervals, same exact recomputation, same
// canonical sums wherever a score can matter); the exact path runs every other shape.
#include "common.h"
#include "indexer_common.h"

namespace {

struct IndexerWs {
  uint16_t *q_rot;
  uint16_t *k_rot;
  float *q_norm;
  int32_t *q_span;
  float *k_norm;
  int32_t *k_span;
  float *scores;
  float *bounds;  // per-score bounds of the bounded path
  float *kmax;    // per key block norm maxima of the bounded path
  uint64_t *part;  // the bounded selection's lists, bucket counts and list lengths
  int64_t part_cap;
  void *w_scaled;  // the head weights times w_scale (ks_indexer_scaled), in the weights' format
  size_t bytes;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

IndexerWs carve(void *base, int64_t B, int64_t S, int64_t H, int64_t D, int64_t T) {
  IndexerWs w{};
  size_t off = 0;
  auto take = [&](size_t n) {
    char *p = base ? static_cast<char *>(base) + off : nullptr;
    off += align256(n);
    return p;
  };
  w.q_rot = reinterpret_cast<uint16_t *>(take(size_t(B * S * H * D) * 2));
  w.k_rot = reinterpret_cast<uint16_t *>(take(size_t(B * T * D) * 2));
  w.q_norm = reinterpret_cast<float *>(take(size_t(B * S * H) * 4));
  w.q_span = reinterpret_cast<int32_t *>(take(size_t(B * S * H) * 4));
  w.k_norm = reinterpret_cast<float *>(take(size_t(B * T) * 4));
  w.k_span = reinterpret_cast<int32_t *>(take(size_t(B * T) * 4));
  w.scores = reinterpret_cast<float *>(take(size_t(B * S * T) * 4));
  w.bounds = reinterpret_cast<float *>(take(size_t(B * S * T) * 4));
  w.kmax = reinterpret_cast<float *>(take(size_t(B * ((T + ks::kScoreKeyBlock - 1) / ks::kScoreKeyBlock)) * 4));
  // the bounded selection's lists and counts (only shapes that can take the bounded path)
  w.part_cap = (H == 64 && D == 128) ? ks::topk_bounded_part_capacity(B * S, T) : 0;
  w.part = reinterpret_cast<uint64_t *>(take(size_t(w.part_cap) * 8));
  w.w_scaled = take(size_t(B * S * H) * 4);
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" size_t ks_indexer_workspace_size(int64_t B, int64_t S, int64_t H, int64_t D, int64_t T) {
  if (B < 0 || S < 0 || H < 0 || D < 0 || T < 0) return 0;
  return carve(nullptr, B, S, H, D, T).bytes;
}

namespace {
// Argument checks shared by the entries (fn names the entry in the messages).
int check_indexer_args(const char *fn, int64_t k_top, int64_t start_pos, int32_t ratio, int64_t B, int64_t S,
                       int64_t H, int64_t D, int64_t T, int64_t k_batch_stride, int path) {
  KS_CHECK_ARG(path >= 0 && path <= 3, "%s: path %d", fn, path);
  KS_CHECK_ARG(D == 128 || D == 64, "%s: D=%lld, the kernels are built for head_dim 64 and 128", fn, (long long)D);
  KS_CHECK_ARG(H == 16 || H == 32 || H == 64, "%s: H=%lld must be 16, 32 or 64", fn, (long long)H);
  KS_CHECK_ARG(B >= 0 && S >= 0, "%s: negative B or S", fn);
  KS_CHECK_ARG(T >= 1 && T <= 65536, "%s: T=%lld must be in [1, 65536]", fn, (long long)T);
  KS_CHECK_ARG(k_batch_stride >= T, "%s: k_batch_stride < T", fn);
  KS_CHECK_ARG(ratio >= 1 && start_pos >= 0, "%s: ratio must be >= 1 and start_pos >= 0", fn);
  KS_CHECK_ARG(k_top >= 1, "%s: k_top must be >= 1", fn);
  const int64_t kk = k_top < T ? k_top : T;
  KS_CHECK_ARG(kk <= 4096, "%s: min(k_top, T)=%lld exceeds 4096", fn, (long long)kk);
  return KS_OK;
}

// Whether the scores take the bounded path (path: 0 = bounded when the shape allows it, 1 = exact, 2 = bounded,
// 3 = bounded with the extended counters).
bool takes_bounded(int64_t k_top, int32_t w_bf16, int64_t H, int64_t D, int64_t T, int path) {
  const int64_t kk = k_top < T ? k_top : T;
  return H == 64 && D == 128 && !w_bf16 && T <= 32768 && kk <= 2048 && path != 1;
}

// The bounded path's count region in the workspace, which the row preparation launch clears when the score
// kernel counts the rows: 16-byte words.
int64_t count_words16(const IndexerWs &ws, int64_t B, int64_t S, int64_t T) {
  return ws.part_cap > 0 && ks::scores_count_rows(B, S, T) ? B * S * ks::kTopkCountWords / 4 : 0;
}

// FP8 keys read directly by the bounded kernels (codes and row scales at batch stride kbs), or none.
struct Fp8Direct {
  const uint8_t *kc = nullptr;
  const float *ks = nullptr;
  int64_t kbs = 0;
};

// Scores of the prepared rows (ws.q_rot / ws.k_rot with their statistics, or the FP8 rows of f8) -> exact top-k.
// Where the score kernel counts the rows, the bounded path needs the count region cleared by the row preparation
// launch.

int indexer_select(const char *fn, const IndexerWs &ws, const void *w, int32_t w_bf16, int64_t k_top, int32_t causal,
                   int64_t start_pos, int32_t ratio, int64_t offset, void *out, int32_t out_i64, int64_t B, int64_t S,
                   int64_t H, int64_t D, int64_t T, hipStream_t st, float bound_c, uint32_t *stats, int path,
                   const Fp8Direct &f8 = Fp8Direct{}, const uint16_t *q_unrot = nullptr, int rot_lo = 0,
                   int rot_hi = 0) {
  const int64_t kk = k_top < T ? k_top : T;
  const bool can_bound = takes_bounded(k_top, w_bf16, H, D, T, 0);
  KS_CHECK_ARG(path < 2 || can_bound,
               "%s: the bounded path needs H = 64, D = 128, fp32 weights, T <= 32768 and k <= 2048", fn);
  int rc;
  if (can_bound && path != 1) {
    const bool counted = ks::scores_count_rows(B, S, T);
    const bool direct = f8.kc != nullptr;
    // FP8 keys: the codes with their row scales (the statistics are indexed like the rows: B == 1 or kbs == T)
    const uint16_t *krows = direct ? reinterpret_cast<const uint16_t *>(f8.kc) : ws.k_rot;
    const int64_t kbs = direct ? f8.kbs : T;
    rc = ks::launch_indexer_scores(ws.q_rot, krows, w, 0, ws.q_norm, ws.q_span, ws.k_norm, ws.k_span, ws.scores, B, S,
                                   H, D, T, kbs, causal ? 1 : 0, start_pos, ratio, bound_c, nullptr, st, ws.bounds,
                                   ws.kmax, counted ? ks::topk_bounded_counts(ws.part, B * S, T) : nullptr, f8.ks);
    if (rc != KS_OK) return rc;
    ks::TopkRecompute trc{ws.bounds, ws.kmax, ws.q_rot, ws.k_rot, static_cast<const float *>(w), ws.q_norm,
                          ws.q_span, ws.k_norm, ws.k_span, kbs, bound_c, stats, path == 3 ? 1 : 0, ws.part,
                          ws.part_cap, counted ? 1 : 0};
    trc.kc = f8.kc;
    trc.ks = f8.ks;
    return ks::launch_indexer_topk_bounded(ws.scores, T, B, S, T, kk, causal ? 1 : 0, start_pos, ratio, offset, out,
                                           out_i64 ? 1 : 0, trc, st);
  }
  // q_unrot: the caller's q rows, whose dims outside [rot_lo, rot_hi) the row preparation did not copy (ws.q_rot
  // then holds only the rotated dims; rot_lo == rot_hi: nothing rotated, all of q from the caller's rows)
  const ks::QSplit qs{rot_hi > rot_lo ? ws.q_rot : nullptr, rot_lo, rot_hi};
  rc = ks::launch_indexer_scores(q_unrot != nullptr ? q_unrot : ws.q_rot, ws.k_rot, w, w_bf16 ? 1 : 0, ws.q_norm,
                                 ws.q_span, ws.k_norm, ws.k_span, ws.scores, B, S, H, D, T, T, causal ? 1 : 0,
                                 start_pos, ratio, bound_c, stats, st, nullptr, nullptr, nullptr, nullptr,
                                 q_unrot != nullptr ? &qs : nullptr);
  if (rc != KS_OK) return rc;
  // bf16 weights: the exact scores are rounded to bf16, so the top-k may take them as bf16 values
  return ks::indexer_topk_impl(ws.scores, T, B, S, T, kk, causal, start_pos, ratio, offset, out, out_i64, st,
                               w_bf16 ? 1 : 0);
}

int indexer_impl(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16, const float *freqs,
                 int64_t freq_rows, int64_t rope_start, int64_t rope_dim, int32_t rope_k, int64_t k_top,
                 int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset, void *out, int32_t out_i64,
                 int64_t B, int64_t S, int64_t H, int64_t D, int64_t T, int64_t k_batch_stride, void *workspace,
                 size_t workspace_bytes, void *stream, float bound_c, uint32_t *stats, int path, float w_scale) {
  ks::last_error().clear();
  int rc = check_indexer_args("ks_indexer", k_top, start_pos, ratio, B, S, H, D, T, k_batch_stride, path);
  if (rc != KS_OK) return rc;
  KS_CHECK_ARG(rope_dim >= 0 && rope_dim % 8 == 0 && rope_start >= 0 && rope_start % 8 == 0 &&
                   rope_start + rope_dim <= D,
               "ks_indexer: rotated segment must be 8-aligned and inside the head");
  if (rope_dim > 0) {
    KS_CHECK_ARG(freqs != nullptr, "ks_indexer: freqs is null");
    KS_CHECK_ARG(start_pos + S <= freq_rows, "ks_indexer: query positions exceed freqs rows");
    KS_CHECK_ARG(!rope_k || T <= freq_rows, "ks_indexer: key positions exceed freqs rows");
  }
  if (B * S == 0) return KS_OK;
  KS_CHECK_ARG(q && k && w && out, "ks_indexer: null pointer");
  KS_CHECK_ARG(ks::aligned(q, 16) && ks::aligned(k, 16), "ks_indexer: q and k must be 16-byte aligned");
  const IndexerWs ws = carve(workspace, B, S, H, D, T);
  KS_CHECK_ARG(workspace != nullptr && workspace_bytes >= ws.bytes,
               "ks_indexer: workspace of %zu bytes required, %zu given", ws.bytes, workspace_bytes);
  KS_CHECK_ARG(ks::aligned(workspace, 256), "ks_indexer: workspace must be 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rd = static_cast<int>(rope_dim);
  // q rows at positions start_pos + s; k rows of every batch (stride k_batch_stride) at positions t
  const bool bounded = takes_bounded(k_top, w_bf16, H, D, T, path);
  // the exact path with a 32-aligned rotated range (or none) reads q's other dims from the caller's rows, so the row
  // preparation writes only the rotated dims of q (half of q's bytes at the drop-in indexer's shape)
  const bool split = !bounded && rope_start % 32 == 0 && rd % 32 == 0;
  ks::RowJob qjob{q, ws.q_rot, ws.q_norm, ws.q_span, B * S * H, B * S * H, B * S * H, H, S, start_pos, rd};
  qjob.rotated_only = split ? 1 : 0;
  const ks::RowJob kjob{k, ws.k_rot, ws.k_norm, ws.k_span, B * T, T, k_batch_stride, 1, T, 0, rope_k ? rd : 0};
  // w_scale != 1: the row preparation also writes the scaled weights (one per q row), which the later launches read
  const bool scaled = w_scale != 1.0f;
  const ks::WeightScale wsc{w, ws.w_scaled, w_scale, w_bf16 ? 1 : 0};
  rc = ks::launch_rope_rows(qjob, kjob, freqs, static_cast<int>(D), static_cast<int>(rope_start), st,
                            bounded ? ks::topk_bounded_counts(ws.part, B * S, T) : nullptr,
                            bounded ? count_words16(ws, B, S, T) : 0, scaled ? &wsc : nullptr);
  if (rc != KS_OK) return rc;
  return indexer_select("ks_indexer", ws, scaled ? ws.w_scaled : w, w_bf16, k_top, causal, start_pos, ratio, offset,
                        out, out_i64, B, S, H, D, T, st, bound_c, stats, path, Fp8Direct{}, split ? q : nullptr,
                        static_cast<int>(rope_start), static_cast<int>(rope_start) + rd);
}

int indexer_fp8_impl(const uint8_t *q, const float *q_scale, const uint8_t *k, const float *k_scale, const void *w,
                     int32_t w_bf16, int64_t k_top, int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset,
                     void *out, int32_t out_i64, int64_t B, int64_t S, int64_t H, int64_t D, int64_t T,
                     int64_t k_batch_stride, void *workspace, size_t workspace_bytes, void *stream, float bound_c,
                     uint32_t *stats, int path) {
  ks::last_error().clear();
  int rc = check_indexer_args("ks_indexer_fp8", k_top, start_pos, ratio, B, S, H, D, T, k_batch_stride, path);
  if (rc != KS_OK) return rc;
  if (B * S == 0) return KS_OK;
  KS_CHECK_ARG(q && q_scale && k && k_scale && w && out, "ks_indexer_fp8: null pointer");
  KS_CHECK_ARG(ks::aligned(q, 8) && ks::aligned(k, 8) && ks::aligned(q_scale, 4) && ks::aligned(k_scale, 4),
               "ks_indexer_fp8: q and k codes must be 8-byte aligned, scales 4-byte aligned");
  const IndexerWs ws = carve(workspace, B, S, H, D, T);
  KS_CHECK_ARG(workspace != nullptr && workspace_bytes >= ws.bytes,
               "ks_indexer_fp8: workspace of %zu bytes required, %zu given", ws.bytes, workspace_bytes);
  KS_CHECK_ARG(ks::aligned(workspace, 256), "ks_indexer_fp8: workspace must be 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bounded = takes_bounded(k_top, w_bf16, H, D, T, path);
  // the bounded kernels read the key codes themselves (their key statistics are indexed like the key rows, so the
  // batches must be contiguous: one batch, or k_batch_stride == T); then this pass forms the keys' statistics only.
  // q is dequantised here in every case: the score kernel reads each query's rows from T / 256 workgroups.
  const bool direct = bounded && (B == 1 || k_batch_stride == T);
  // q rows (scale per row) and k rows of every batch (stride k_batch_stride, scale per row, same stride)
  const ks::Fp8RowJob qjob{q, q_scale, ws.q_rot, ws.q_norm, ws.q_span, B * S * H, B * S * H, B * S * H};
  const ks::Fp8RowJob kjob{k, k_scale, direct ? nullptr : ws.k_rot, ws.k_norm, ws.k_span, B * T, T, k_batch_stride};
  rc = ks::launch_fp8_rows(qjob, kjob, static_cast<int>(D), st,
                           bounded ? ks::topk_bounded_counts(ws.part, B * S, T) : nullptr,
                           bounded ? count_words16(ws, B, S, T) : 0);
  if (rc != KS_OK) return rc;
  Fp8Direct f8;
  if (direct) {
    f8.kc = k;
    f8.ks = k_scale;
    f8.kbs = k_batch_stride;
  }
  return indexer_select("ks_indexer_fp8", ws, w, w_bf16, k_top, causal, start_pos, ratio, offset, out, out_i64, B, S,
                        H, D, T, st, bound_c, stats, path, f8);
}
}  // namespace

extern "C" int ks_indexer(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16, const float *freqs,
                          int64_t freq_rows, int64_t rope_start, int64_t rope_dim, int32_t rope_k, int64_t k_top,
                          int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset, void *out,
                          int32_t out_i64, int64_t B, int64_t S, int64_t H, int64_t D, int64_t T,
                          int64_t k_batch_stride, void *workspace, size_t workspace_bytes, void *stream) {
  return indexer_impl(q, k, w, w_bf16, freqs, freq_rows, rope_start, rope_dim, rope_k, k_top, causal, start_pos, ratio,
                      offset, out, out_i64, B, S, H, D, T, k_batch_stride, workspace, workspace_bytes, stream,
                      ks::score_bound_c(D), nullptr, 0, 1.0f);
}

extern "C" int ks_indexer_scaled(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16,
                                 float w_scale, const float *freqs, int64_t freq_rows, int64_t rope_start,
                                 int64_t rope_dim, int32_t rope_k, int64_t k_top, int32_t causal, int64_t start_pos,
                                 int32_t ratio, int64_t offset, void *out, int32_t out_i64, int64_t B, int64_t S,
                                 int64_t H, int64_t D, int64_t T, int64_t k_batch_stride, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(__builtin_isfinite(w_scale), "ks_indexer_scaled: w_scale must be finite");
  return indexer_impl(q, k, w, w_bf16, freqs, freq_rows, rope_start, rope_dim, rope_k, k_top, causal, start_pos, ratio,
                      offset, out, out_i64, B, S, H, D, T, k_batch_stride, workspace, workspace_bytes, stream,
                      ks::score_bound_c(D), nullptr, 0, w_scale);
}

// Diagnostic variant (not part of the public header): explicit error-bound constant, path choice (0 auto,
// 1 exact, 2 bounded, 3 bounded with a third counter) and device counters stats[0] += exact dot
// recomputations, stats[1] += dots outside the provably exact range (path 3: stats[2] += recomputed scores).
extern "C" int ks_dbg_indexer(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16, const float *freqs,
                              int64_t freq_rows, int64_t rope_start, int64_t rope_dim, int32_t rope_k, int64_t k_top,
                              int32_t causal, int64_t start_pos, int32_t ratio, int64_t offset, void *out,
                              int32_t out_i64, int64_t B, int64_t S, int64_t H, int64_t D, int64_t T,
                              int64_t k_batch_stride, void *workspace, size_t workspace_bytes, void *stream,
                              float bound_c, uint32_t *stats, int32_t path) {
  return indexer_impl(q, k, w, w_bf16, freqs, freq_rows, rope_start, rope_dim, rope_k, k_top, causal, start_pos, ratio,
                      offset, out, out_i64, B, S, H, D, T, k_batch_stride, workspace, workspace_bytes, stream, bound_c,
                      stats, path, 1.0f);
}

extern "C" int ks_indexer_fp8(const uint8_t *q, const float *q_scale, const uint8_t *k, const float *k_scale,
                              const void *w, int32_t w_bf16, int64_t k_top, int32_t causal, int64_t start_pos,
                              int32_t ratio, int64_t offset, void *out, int32_t out_i64, int64_t B, int64_t S,
                              int64_t H, int64_t D, int64_t T, int64_t k_batch_stride, void *workspace,
                              size_t workspace_bytes, void *stream) {
  return indexer_fp8_impl(q, q_scale, k, k_scale, w, w_bf16, k_top, causal, start_pos, ratio, offset, out, out_i64, B,
                          S, H, D, T, k_batch_stride, workspace, workspace_bytes, stream, ks::score_bound_c(D), nullptr,
                          0);
}

// Diagnostic variant of ks_indexer_fp8 with the path choice and counters of ks_dbg_indexer.
extern "C" int ks_dbg_indexer_fp8(const uint8_t *q, const float *q_scale, const uint8_t *k, const float *k_scale,
                                  const void *w, int32_t w_bf16, int64_t k_top, int32_t causal, int64_t start_pos,
                                  int32_t ratio, int64_t offset, void *out, int32_t out_i64, int64_t B, int64_t S,
                                  int64_t H, int64_t D, int64_t T, int64_t k_batch_stride, void *workspace,
                                  size_t workspace_bytes, void *stream, uint32_t *stats, int32_t path) {
  return indexer_fp8_impl(q, q_scale, k, k_scale, w, w_bf16, k_top, causal, start_pos, ratio, offset, out, out_i64, B,
                          S, H, D, T, k_batch_stride, workspace, workspace_bytes, stream, ks::score_bound_c(D), stats,
                          path);
}
