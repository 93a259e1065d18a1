/*
 * kswift.h — C ABI of the MI355X (gfx950) KernelSwift operator library
 * (libkswift_amd.so).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as void*, enqueues its kernels on that stream and returns without
 * synchronising.  No torch type appears in any signature; callers (the Python
 * host layer in kernelswift_amd/ops.py, or a ctypes / C++ binding) own all
 * memory.  Return value: KS_OK, or an error code with a message readable from
 * ks_last_error() (thread-local).  Argument errors are detected on the host
 * before anything is enqueued, mirroring the TORCH_CHECK validation of the
 * reference's torch extensions; there is no fallback path.
 *
 * Element types: "bf16" buffers hold raw bfloat16 bit patterns (uint16_t),
 * "f32" buffers IEEE binary32, index buffers int32 or int64 as stated.
 * All tensors are dense row-major (C-contiguous) unless a leading dimension
 * argument says otherwise.
 */
#ifndef KSWIFT_H
#define KSWIFT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KS_OK 0
#define KS_ERR_INVALID 1 /* argument validation failed (shape, size, alignment, null) */
#define KS_ERR_HIP 2     /* a HIP runtime call or kernel launch failed */

/* Message of the last failing call on this thread ("" if none). */
const char *ks_last_error(void);

/* Library ABI version (major*100 + minor). */
int ks_version(void);

/* ------------------------------------------------------------------------
 * Sinkhorn normalisation of a batch of 4x4 fp32 matrices.
 *
 * Replaces the reference kernel stub
 *   sinkhorn_kernel(blockDim, l2Ctrl, stream, x, out, total_matrices, repeat, eps)
 *   (optimized/sinkhorn_project/op_extension/sinkhorn_torch.cpp:13-16)
 * behind the op sinkhorn_torch(x, repeat, eps) (sinkhorn_torch.cpp:18), with
 * the semantics of baseline/sinkhorn.py:13-19:
 *   x = softmax(x, -1) + eps;  x /= colsum(x) + eps;
 *   repeat-1 times { x /= rowsum(x) + eps;  x /= colsum(x) + eps; }
 * x, out: f32 [n_mats, 4, 4]; out may not alias x.  n_mats may be 0.
 * repeat >= 1.  Unlike the reference stub there is no upper bound on n_mats.
 * ---------------------------------------------------------------------- */
int ks_sinkhorn(const float *x, float *out, int64_t n_mats, int32_t repeat,
                float eps, void *stream);

/* ------------------------------------------------------------------------
 * Rotary embedding, in place, on bf16 rows.
 *
 * Replaces indexer_rope_kernel(blockDim, l2Ctrl, stream, q, freqs, b, s, h, d, pairs)
 *   (optimized/indexer_project/op_extension/indexer_torch.cpp:51-53)
 * behind rope_inplace(q, freqs) (indexer_torch.cpp:174), semantics of
 * apply_rotary_emb (baseline/indexer.py:114-129): consecutive pairs
 * (2j, 2j+1) of the rotated segment are multiplied, as complex numbers, by
 * (cos, sin) of the token's position, in fp32, and rounded back to bf16 (RNE).
 * Canonical arithmetic (no fused multiply-add):
 *   y0 = bf16( fl(x0*c) - fl(x1*s) ),  y1 = bf16( fl(x0*s) + fl(x1*c) ).
 *
 * x:     bf16 [B, S, H, D]
 * freqs: f32  [freq_rows, rope_dim/2, 2]   (cos, sin) per pair: the real view of
 *        the complex freqs_cis table of baseline/indexer.py:226-235.
 * Token (b, s) uses freqs row pos0 + s; requires pos0 + S <= freq_rows.
 * The rotated segment is dims [rope_start, rope_start + rope_dim) of each
 * head row; rope_dim even, rope_start + rope_dim <= D.
 * ---------------------------------------------------------------------- */
int ks_rope_inplace(uint16_t *x, const float *freqs, int64_t B, int64_t S,
                    int64_t H, int64_t D, int64_t rope_start, int64_t rope_dim,
                    int64_t pos0, int64_t freq_rows, void *stream);

/* ------------------------------------------------------------------------
 * Indexer scores: score[b,s,t] = sum_h w[b,s,h] * relu(bf16(q[b,s,h,:] . k[b,t,:]))
 * plus the causal mask.
 *
 * Replaces fused_indexer_qk_reduce(blockDim, l2Ctrl, stream, q, kvT, weights, out,
 *   scores, ...) (optimized/indexer_project/op_extension/indexer_torch.cpp:43-50)
 * behind fused_qk_reduce(q, kvT, weights, causal, ratio) (indexer_torch.cpp:100),
 * generalised to the semantics of baseline/indexer.py:176-193 at any H, any
 * start position and fp32 or bf16 head weights.  k is read untransposed.
 *
 * Canonical arithmetic (bit-exact contract):
 *   d_h   = the exact real dot product of the bf16 vectors, rounded once to bf16 (RNE);
 *   r_h   = max(d_h, 0);
 *   w_bf16 == 0 (fp32 weights):  p_h = r_h * w_h            (fp32, fused into the add below)
 *   group sums G_g, g = 0..3, over heads h with (h/4) % 4 == g in increasing h:
 *         G_g = fma(r_h, w_h, G_g) from G_g = +0        (fp32 weights)
 *         G_g = G_g + bf16(r_h * w_h)                   (bf16 weights)
 *   score = (G_0 + G_1) + (G_2 + G_3), rounded to bf16 when w_bf16 != 0.
 *   Causal (causal != 0): query s sits at position start_pos + s and sees keys
 *   t < (start_pos + s + 1) / ratio (integer division); others score -inf.
 *
 * q: bf16 [B, S, H, D];  k: bf16, batch b's T rows start at k + b*k_batch_stride*D
 * (k_batch_stride >= T rows);  w: [B, S, H] f32 (w_bf16 == 0) or bf16.
 * q_norm/q_span: [B*S*H] and k_norm/k_span: [B*k_batch_stride] row statistics
 * from ks_indexer_row_stats over the same q and k buffers (they bound the MFMA
 * error and prove the exact recomputation of near-tie dots exact).
 * scores: f32 [B, S, T].  D must be 64 or 128 (the head dims the kernel is
 * built for); H in {16, 32, 64}; T >= 1.
 * Exact for all finite inputs: the MFMA sum is trusted only when an interval of
 * half-width C * 2^-23 * (||q|| + 2^-122)(||k|| + 2^-122) + 2^-144 around it
 * rounds to one bf16 value (C = 13 for D = 128, 9 for D = 64: a bound derived
 * from the instruction's accumulation over D / 8 steps);
 * other dots are recomputed exactly (double precision, or an integer accumulator
 * for rows of any dynamic range), and rows whose norm product reaches 2^126 are
 * recomputed in full.  Scores must not come out NaN (an infinite dot times a zero
 * weight, or opposite infinities); NaN and infinite inputs are outside the contract.
 * ---------------------------------------------------------------------- */
int ks_indexer_scores(const uint16_t *q, const uint16_t *k, const void *w,
                      int32_t w_bf16, const float *q_norm, const int32_t *q_span,
                      const float *k_norm, const int32_t *k_span, float *scores,
                      int64_t B, int64_t S, int64_t H, int64_t D, int64_t T,
                      int64_t k_batch_stride, int32_t causal, int64_t start_pos,
                      int32_t ratio, void *stream);

/* ------------------------------------------------------------------------
 * Per-row statistics of bf16 rows of length D (64 or 128) for ks_indexer_scores:
 *   norm[r] >= ||x_r||_2 (an upper bound within 2^-11 relative),
 *   span[r]  = ceil(log2 norm[r]) - (exponent of the least significant bit of
 *              the smallest nonzero element), 0 for an all-zero row.
 * No reference counterpart: the reference kernel had no exactness contract.
 * ---------------------------------------------------------------------- */
int ks_indexer_row_stats(const uint16_t *x, int64_t rows, int64_t D, float *norm,
                         int32_t *span, void *stream);

/* ------------------------------------------------------------------------
 * Fused indexer: RoPE -> scores -> top-k, the three-op sequence of the
 * reference wrapper (optimized/indexer_project/indexer.py:197-222:
 * rope_inplace, fused_qk_reduce, topk_mask) behind one call, with the
 * semantics of baseline/indexer.py:161-206 after the projections.
 * q is rotated at positions start_pos + s, k (when rope_k != 0) at positions t,
 * both over dims [rope_start, rope_start + rope_dim) with the freqs table of
 * ks_rope_inplace; inputs are not modified (rotated copies live in the
 * workspace).  out: [B*S, min(k_top, T)] int32 or int64 (out_i64), as
 * ks_indexer_topk.  workspace: ks_indexer_workspace_size(B, S, H, D, T) bytes,
 * 256-byte aligned.  Shapes as ks_indexer_scores: q bf16 [B, S, H, D] with
 * D in {64, 128} and H in {16, 32, 64}; batch b's T key rows start at
 * k + b*k_batch_stride*D; w [B, S, H]; T <= 65536.
 * With H = 64, D = 128, fp32 weights, T <= 32768 and min(k_top, T) <= 2048
 * the scores are computed with per-score bounds and only the scores that can
 * reach the top k are recomputed exactly (inside the top-k kernel); the
 * returned indices are those of the exact path.
 * ---------------------------------------------------------------------- */
size_t ks_indexer_workspace_size(int64_t B, int64_t S, int64_t H, int64_t D,
                                 int64_t T);
int ks_indexer(const uint16_t *q, const uint16_t *k, const void *w, int32_t w_bf16,
               const float *freqs, int64_t freq_rows, int64_t rope_start,
               int64_t rope_dim, int32_t rope_k, int64_t k_top, int32_t causal,
               int64_t start_pos, int32_t ratio, int64_t offset, void *out,
               int32_t out_i64, int64_t B, int64_t S, int64_t H, int64_t D,
               int64_t T, int64_t k_batch_stride, void *workspace,
               size_t workspace_bytes, void *stream);
/* The same with the head weights multiplied by w_scale on the way, as the
 * reference's caller computes weights_proj(x) * (softmax_scale * n_heads^-0.5)
 * (baseline/indexer.py:174-175) before the indexer: each weight becomes
 * fp32(w * fp32(w_scale)), rounded to bf16 (nearest even) for bf16 weights,
 * which is torch's rounding of a tensor times a Python float; the scaled
 * weights live in the workspace, the input is not modified.  w_scale finite. */
int ks_indexer_scaled(const uint16_t *q, const uint16_t *k, const void *w,
                      int32_t w_bf16, float w_scale, const float *freqs,
                      int64_t freq_rows, int64_t rope_start, int64_t rope_dim,
                      int32_t rope_k, int64_t k_top, int32_t causal,
                      int64_t start_pos, int32_t ratio, int64_t offset, void *out,
                      int32_t out_i64, int64_t B, int64_t S, int64_t H, int64_t D,
                      int64_t T, int64_t k_batch_stride, void *workspace,
                      size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * FP8 block quantisation of bf16 rows (e4m3fn codes, one fp32 scale per block),
 * for the quantised indexer of the reference's dtype = "fp8",
 * scale_fmt = "ue8m0" configuration (baseline/indexer.py:14-17; the reference
 * names the format but ships no kernel for it).  Per block of `block` elements
 * of a row:
 *   amax = max(max|x|, 1e-4);  s = amax * fp32(1/448)  (fp32, nearest even);
 *   ue8m0 != 0: s = 2^ceil(log2 s)  (a power of two);
 *   code = e4m3fn(clamp(x / s, -448, 448)), nearest even (IEEE division).
 * x: bf16 [rows, D] (16-byte aligned); codes: [rows, D] bytes (8-byte aligned);
 * scales: f32 [rows, D / block].  block in {8, 16, 32, 64, 128}, D % block == 0.
 * Finite inputs only.
 * ---------------------------------------------------------------------- */
int ks_fp8_quant_rows(const uint16_t *x, int64_t rows, int64_t D, int64_t block,
                      int32_t ue8m0, uint8_t *codes, float *scales, void *stream);

/* ------------------------------------------------------------------------
 * Indexer on FP8 rows: scores -> top-k of ks_indexer (same contract, same
 * exactness, same output) on the dequantised rows
 *   q_h[d] = bf16(fp32(e4m3(q codes[d]) * q_scale)),  likewise k,
 * one scale per row (a whole head of D elements: block = D in
 * ks_fp8_quant_rows); with power-of-two (ue8m0) scales the dequantised values
 * are exactly code * scale.  No RoPE: quantised rows are stored after it.
 * q: [B, S, H, D] codes, q_scale: f32 [B, S, H]; k: batch b's T key rows of D
 * codes start at k + b*k_batch_stride*D, k_scale: f32, batch b's scales start at
 * k_scale + b*k_batch_stride.  Codes 8-byte aligned; no NaN codes.  Shapes,
 * weights, outputs and workspace (ks_indexer_workspace_size) as ks_indexer.
 * No reference counterpart (an FP8 configuration of baseline/indexer.py:14-17
 * over the scoring of baseline/indexer.py:191-206).
 * ---------------------------------------------------------------------- */
int ks_indexer_fp8(const uint8_t *q, const float *q_scale, const uint8_t *k,
                   const float *k_scale, const void *w, int32_t w_bf16,
                   int64_t k_top, int32_t causal, int64_t start_pos, int32_t ratio,
                   int64_t offset, void *out, int32_t out_i64, int64_t B, int64_t S,
                   int64_t H, int64_t D, int64_t T, int64_t k_batch_stride,
                   void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * Exact sorted top-k per row with the reference post-processing.
 *
 * Replaces indexer_topk_kernel(blockDim, l2Ctrl, stream, scores, out, totalRows,
 *   rowsPerCore, seqlen, causal, ratio, actualT, offset, tiling...)
 *   (optimized/indexer_project/op_extension/indexer_torch.cpp:54-58)
 * behind topk_mask(scores, causal, ratio, actualT, offset) (indexer_torch.cpp:232),
 * semantics of baseline/indexer.py:195-206:
 *   idx[r, 0..k) = the k columns of row r with the largest scores, ordered by
 *   (score descending, column ascending) — i.e. a stable descending sort's
 *   prefix (-inf sorts last, lowest column first among equal scores);
 *   causal != 0: idx >= (start_pos + s + 1)/ratio  ->  -1, else idx + offset
 *   causal == 0: idx + offset.
 * Rows are r = b*S + s.  scores: f32 [B*S rows, ld] (first T columns used,
 * NaN not allowed).  out: [B*S, k] int32 (out_i64 == 0) or int64.
 * 1 <= k <= min(T, 4096), T <= 65536.
 * ---------------------------------------------------------------------- */
int ks_indexer_topk(const float *scores, int64_t ld, int64_t B, int64_t S,
                    int64_t T, int64_t k, int32_t causal, int64_t start_pos,
                    int32_t ratio, int64_t offset, void *out, int32_t out_i64,
                    void *stream);

/* ------------------------------------------------------------------------
 * Sparse attention over gathered top-k KV rows with an attention sink.
 *
 * Replaces fused_sparse_attn_basic_kernel(blockDim, l2Ctrl, stream, q, kv, kvT,
 *   sink, topk, scores, agg, out, tiling) and transpose_kv_kernel
 *   (optimized/sparse_attention/op_extension/sparse_attn_torch.cpp:45-48)
 * behind sparse_attn_megakernel_basic(q, kv, attn_sink, topk_idxs, softmax_scale)
 *   (optimized/sparse_attention/op_extension/register.cpp:9-10),
 * semantics of sparse_attn_ref (baseline/sparse_attention.py:5-42):
 *   s[h,t] = scale * q[b,m,h,:Dqk] . kv[b, idx[b,m,t], :Dqk]   (idx >= 0 only)
 *   z = max(max_t s, sink[h]); e_t = exp(s - z); den = sum e + exp(sink - z)
 *   out[b,m,h,:Dv] = sum_t (e_t/den) kv[b, idx[b,m,t], :Dv]   (bf16 output)
 * Negative indices are invalid (contribute nothing); duplicates count with
 * multiplicity.  Dv <= Dqk (V is the first Dv columns of kv).
 * q: bf16 [B, M, H, Dqk]; kv: bf16 [B, N, Dqk]; sink: f32 [H];
 * idx: int32 [B, M, K]; out: bf16 [B, M, H, Dv].
 * workspace: device buffer of ks_sparse_attn_workspace_size(...) bytes
 * (may be NULL when that size is 0).  Indices >= N are an error the kernel
 * cannot report; they are treated as invalid (masked), never dereferenced.
 * ---------------------------------------------------------------------- */
size_t ks_sparse_attn_workspace_size(int64_t B, int64_t M, int64_t H,
                                     int64_t Dqk, int64_t Dv, int64_t K);
int ks_sparse_attn(const uint16_t *q, const uint16_t *kv, const float *sink,
                   const int32_t *idx, uint16_t *out, int64_t B, int64_t M,
                   int64_t H, int64_t Dqk, int64_t Dv, int64_t N, int64_t K,
                   float scale, void *workspace, size_t workspace_bytes,
                   void *stream);

/* ------------------------------------------------------------------------
 * mHC residual hyper-connections (hc_mult = 4 streams) with the Sinkhorn
 * projection fused into the mixing that consumes it.
 *
 * No kernel counterpart in the reference: it configures hc_mult = 4,
 * hc_sinkhorn_iters = 20 and hc_eps (baseline/indexer.py:48-50) and ships the
 * 4x4 Sinkhorn as an operator of its own (baseline/sinkhorn.py, mhc = 4 there;
 * ks_sinkhorn above).  Per token t, with residual streams x[t] (4 rows of C):
 *   ks_mhc_pre:  h[t]    = sum_j sigmoid(pre_logits[t][j]) x[t][j]
 *   ks_mhc_post: out[t][i] = sum_j S(res_logits[t])[i][j] x[t][j]
 *                           + 2 sigmoid(post_logits[t][i]) f[t]
 * where S is the Sinkhorn of ks_sinkhorn (repeat = sinkhorn_iters, eps) of the
 * token's 4x4 logits, computed inside the kernel (the matrices never reach
 * memory).  x: bf16 [N, 4, C], C a multiple of 8; f, h: bf16 [N, C];
 * pre_logits, post_logits: f32 [N, 4]; res_logits: f32 [N, 4, 4];
 * out: bf16 [N, 4, C], may alias x.  fp32 arithmetic, RNE to bf16; every
 * buffer 16-byte aligned.
 * ---------------------------------------------------------------------- */
int ks_mhc_pre(const uint16_t *x, const float *pre_logits, uint16_t *h, int64_t N,
               int64_t C, void *stream);
int ks_mhc_post(const uint16_t *x, const uint16_t *f, const float *res_logits,
                const float *post_logits, uint16_t *out, int64_t N, int64_t C,
                int32_t sinkhorn_iters, float eps, void *stream);

/* ------------------------------------------------------------------------
 * ks_sparse_attn without a workspace: allocates nothing.
 *
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments and results as ks_sparse_attn, minus the workspace:
 * the split partials live in a static device array of
 * ks_sparse_attn_noalloc_max_scratch() bytes (64 MiB).  The array is part of the
 * library's code object, so every GPU on which the library is loaded holds its own
 * 64 MiB copy for the life of the process, whether or not this entry point is ever
 * called.  Its address on the stream's device is resolved (hipGetSymbolAddress) on
 * that device's first call: make one call on each device before capturing this
 * entry point into a HIP graph, so that the capture records kernel launches only.
 * Shapes whose ks_sparse_attn_workspace_size exceeds the maximum return
 * KS_ERR_INVALID without launching.  Calls that overlap on one GPU (two streams,
 * two threads) share the array and race: serialise them.  The array keeps the last
 * call's contents; no call relies on them (every partial is written before it is
 * read within the call).
 * ---------------------------------------------------------------------- */
size_t ks_sparse_attn_noalloc_max_scratch(void);
int ks_sparse_attn_noalloc(const uint16_t *q, const uint16_t *kv, const float *sink,
                           const int32_t *idx, uint16_t *out, int64_t B, int64_t M,
                           int64_t H, int64_t Dqk, int64_t Dv, int64_t N, int64_t K,
                           float scale, void *stream);

/* ------------------------------------------------------------------------
 * Calibration helper (not an operator): copies n_bytes (multiple of 16) from
 * src to dst with one streaming kernel.  Used to scale rocprofv3 FETCH_SIZE /
 * WRITE_SIZE counters against a kernel of known traffic.
 * ---------------------------------------------------------------------- */
int ks_copy_bytes(const void *src, void *dst, int64_t n_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KSWIFT_H */
