"""Torch-facing operators over the C ABI of libkswift_amd.so.

Each function mirrors one op of the reference's torch extensions (same name or
the reference name in the docstring, same argument meaning, RuntimeError on
invalid input like TORCH_CHECK) and launches the gfx950 kernels on the current
HIP stream without synchronising.  PyTorch only provides device memory and the
stream; there is no CPU or torch fallback: a tensor on the wrong device, a
missing library or an unsupported shape raises.
"""
from __future__ import annotations

import ctypes
import functools
from typing import Optional

import torch

from . import _lib

__all__ = [
    "sinkhorn", "rope_inplace", "indexer_row_stats", "indexer_scores", "topk_mask", "indexer",
    "indexer_workspace_size", "fp8_quant", "indexer_fp8", "sparse_attn", "sparse_attn_workspace_size", "mhc_pre",
    "mhc_post", "copy_bytes",
]


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(*ts: torch.Tensor, contiguous: bool = True) -> None:
    for t in ts:
        _check(t.is_cuda, "tensors must be on the GPU (there is no CPU path)")
        _check(not contiguous or t.is_contiguous(), "tensors must be contiguous")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """The current HIP stream of t's device as a raw handle (torch's raw query when present: it skips building
    a Stream object on every call, which host-bound small launches pay for)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------- Sinkhorn
def sinkhorn(x: torch.Tensor, repeat: int = 10, eps: float = 1e-6) -> torch.Tensor:
    """sinkhorn_torch(x, repeat, eps) (optimized/sinkhorn_project/op_extension/sinkhorn_torch.cpp:18).

    x: float32 [..., 4, 4] (any leading dims; the reference required 4-D and <= 2560 matrices).
    Returns a new tensor (out-of-place, like the reference's empty_like output)."""
    _check(x.dtype == torch.float32, "x must be float32")
    _on_gpu(x)
    _check(x.dim() >= 2 and x.shape[-1] == 4 and x.shape[-2] == 4, "x must be [..., 4, 4]")
    _check(repeat >= 1, "repeat must be >= 1")
    out = torch.empty_like(x)
    n = x.numel() // 16
    _lib.check(_lib.load().ks_sinkhorn(_p(x), _p(out), n, int(repeat), float(eps), _stream(x)), "sinkhorn")
    return out


# ---------------------------------------------------------------- indexer
def rope_inplace(x: torch.Tensor, freqs: torch.Tensor, rope_start: Optional[int] = None, rope_dim: Optional[int] = None,
                 pos0: int = 0) -> None:
    """rope_inplace(q, freqs) (optimized/indexer_project/op_extension/indexer_torch.cpp:174).

    x: bf16 [B, S, H, D] or [B, S, D], rotated in place.  freqs: float32 [rows, P, 2] (cos, sin), the real
    view of freqs_cis.  Default segment = the trailing 2P dims (the reference op's choice); pass
    rope_start=0 for the leading dims.  Token s uses freqs row pos0 + s."""
    _check(x.dtype == torch.bfloat16, "x must be bfloat16")
    _check(freqs.dtype == torch.float32 and freqs.dim() == 3 and freqs.shape[2] == 2, "freqs must be float32 [s, p, 2]")
    _on_gpu(x, freqs)
    _check(x.dim() in (3, 4), "x must be [b, s, h, d] or [b, s, d]")
    B, S = x.shape[0], x.shape[1]
    H = x.shape[2] if x.dim() == 4 else 1
    D = x.shape[-1]
    P = freqs.shape[1]
    rd = 2 * P if rope_dim is None else rope_dim
    _check(rd == 2 * P, "rope_dim must equal 2 * freqs.shape[1]")
    rs = D - rd if rope_start is None else rope_start
    _lib.check(_lib.load().ks_rope_inplace(_p(x), _p(freqs), B, S, H, D, rs, rd, pos0, freqs.shape[0], _stream(x)),
               "rope_inplace")


def indexer_row_stats(x: torch.Tensor):
    """Row statistics (norm upper bound, span) of bf16 rows of length 64 or 128 for indexer_scores."""
    _check(x.dtype == torch.bfloat16 and x.shape[-1] in (64, 128), "x must be bfloat16 [..., 64 or 128]")
    _check(x.is_contiguous(), "x must be contiguous")
    _on_gpu(x)
    D = x.shape[-1]
    rows = x.numel() // D
    norm = torch.empty(rows, dtype=torch.float32, device=x.device)
    span = torch.empty(rows, dtype=torch.int32, device=x.device)
    _lib.check(_lib.load().ks_indexer_row_stats(_p(x), rows, D, _p(norm), _p(span), _stream(x)), "indexer_row_stats")
    return norm, span


def indexer_scores(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor, causal: bool, start_pos: int = 0,
                   ratio: int = 1, T: Optional[int] = None, stats=None) -> torch.Tensor:
    """fused_qk_reduce(q, kvT, weights, causal, ratio) (indexer_torch.cpp:100), generalised.

    q: bf16 [B, S, H, D] (already rotated, D = 64 or 128); k: bf16 [B, Tk, D] contiguous (untransposed,
    first T rows used);
    weights: float32 or bf16 [B, S, H].  Returns float32 scores [B, S, T] with -inf where masked.
    stats: optional ((q_norm, q_span), (k_norm, k_span)) from indexer_row_stats."""
    _check(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16, "q and k must be bfloat16")
    _check(weights.dtype in (torch.float32, torch.bfloat16), "weights must be float32 or bfloat16")
    _on_gpu(q, k, weights)
    _check(q.dim() == 4 and k.dim() == 3 and weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]")
    B, S, H, D = q.shape
    _check(k.shape[0] == B and k.shape[2] == D, "k shape mismatch")
    _check(tuple(weights.shape) == (B, S, H), "weights shape mismatch")
    _check(q.is_contiguous() and k.is_contiguous() and weights.is_contiguous(), "q, k, weights must be contiguous")
    Tk = k.shape[1]
    T = Tk if T is None else T
    if stats is None:
        stats = (indexer_row_stats(q), indexer_row_stats(k))
    (qn, qs), (kn, ks_) = stats
    out = torch.empty((B, S, T), dtype=torch.float32, device=q.device)
    _lib.check(_lib.load().ks_indexer_scores(_p(q), _p(k), _p(weights), 1 if weights.dtype == torch.bfloat16 else 0,
                                             _p(qn), _p(qs), _p(kn), _p(ks_), _p(out), B, S, H, D, T, Tk,
                                             1 if causal else 0, start_pos, ratio, _stream(q)), "indexer_scores")
    return out


def topk_mask(scores: torch.Tensor, causal: bool, ratio: int, actual_t: int, offset: int, k: int = 128,
              start_pos: int = 0, out_dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """topk_mask(scores, causal, ratio, actualT, offset) (indexer_torch.cpp:232), generalised.

    scores: float32 [B, S, ld] (first actual_t columns used).  Returns [B, S, min(k, actual_t)] indices
    sorted by (score desc, column asc); causal: column >= (start_pos+s+1)//ratio -> -1, else +offset."""
    _check(scores.dtype == torch.float32, "scores must be float32")
    _on_gpu(scores)
    _check(scores.dim() == 3, "scores must be [b, s, t]")
    _check(out_dtype in (torch.int32, torch.int64), "out_dtype must be int32 or int64")
    B, S, ld = scores.shape
    kk = min(k, actual_t)
    out = torch.empty((B, S, kk), dtype=out_dtype, device=scores.device)
    _lib.check(_lib.load().ks_indexer_topk(_p(scores), ld, B, S, actual_t, kk, 1 if causal else 0, start_pos, ratio,
                                           offset, _p(out), 1 if out_dtype == torch.int64 else 0, _stream(scores)),
               "topk_mask")
    return out


@functools.lru_cache(maxsize=256)  # a pure function of the shape: cached so that calls pay no C round trip
def indexer_workspace_size(B: int, S: int, H: int, D: int, T: int) -> int:
    return int(_lib.load().ks_indexer_workspace_size(B, S, H, D, T))


def indexer(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor, freqs: Optional[torch.Tensor], k_top: int,
            causal: bool, start_pos: int, ratio: int = 1, offset: int = 0, rope_start: int = 0, rope_dim: int = 64,
            rope_k: bool = True, out_dtype: torch.dtype = torch.int32,
            workspace: Optional[torch.Tensor] = None, T: Optional[int] = None, w_scale: float = 1.0) -> torch.Tensor:
    """Fused RoPE -> exact scores -> exact top-k (the reference wrapper's three-op sequence,
    optimized/indexer_project/indexer.py:197-222).  Inputs are not modified.  w_scale: the weights are used as
    weights * w_scale with torch's rounding (ks_indexer_scaled), without a separate multiply.

    q: bf16 [B, S, H, D] (D = 64 or 128); k: bf16 [B, Tk, D] whose rows are contiguous (a batch-strided view
    such as kv_cache[:B] is accepted without a copy), the first T (default Tk) rows are the keys;
    weights float32/bf16 [B, S, H]; freqs: float32 [rows, rope_dim/2, 2].
    Returns [B, S, min(k_top, T)] int32 (default) or int64."""
    _check(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16, "q and k must be bfloat16")
    _check(weights.dtype in (torch.float32, torch.bfloat16), "weights must be float32 or bfloat16")
    _on_gpu(q, weights)
    _on_gpu(k, contiguous=False)  # batch-strided rows allowed, checked below
    _check(q.dim() == 4 and k.dim() == 3 and weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]")
    B, S, H, D = q.shape
    _check(k.shape[0] >= B and k.shape[2] == D, "k shape mismatch")
    _check(tuple(weights.shape) == (B, S, H), "weights shape mismatch")
    _check(q.is_contiguous() and weights.is_contiguous(), "q and weights must be contiguous")
    _check(k.stride(2) == 1 and k.stride(1) == D and k.stride(0) % D == 0, "k rows must be contiguous")
    T = k.shape[1] if T is None else T
    _check(1 <= T <= k.shape[1], "T out of range")
    kbs = k.stride(0) // D if B > 1 else max(k.shape[1], T)
    if rope_dim > 0:
        _check(freqs is not None and freqs.dtype == torch.float32 and freqs.shape[1] * 2 == rope_dim,
               "freqs must be float32 [rows, rope_dim/2, 2]")
        _on_gpu(freqs)
    need = indexer_workspace_size(B, S, H, D, T)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    kk = min(k_top, T)
    out = torch.empty((B, S, kk), dtype=out_dtype, device=q.device)
    fr = freqs.shape[0] if freqs is not None else 0
    _lib.check(_lib.load().ks_indexer_scaled(_p(q), _p(k), _p(weights), 1 if weights.dtype == torch.bfloat16 else 0,
                                             float(w_scale), _p(freqs), fr, rope_start, rope_dim, 1 if rope_k else 0,
                                             k_top, 1 if causal else 0, start_pos, ratio, offset, _p(out),
                                             1 if out_dtype == torch.int64 else 0, B, S, H, D, T, kbs, _p(workspace),
                                             workspace.numel(), _stream(q)), "indexer")
    return out


def fp8_quant(x: torch.Tensor, block: int = 128, ue8m0: bool = True):
    """FP8 block quantisation of bf16 rows (the dtype = "fp8", scale_fmt = "ue8m0" configuration of
    baseline/indexer.py:14-17): per block of `block` elements of the last dim, s = max(amax, 1e-4) * fp32(1/448)
    (a power of two 2^ceil(log2 s) under ue8m0), codes = e4m3fn(clamp(x / s, -448, 448)) nearest even.

    x: bf16 [..., D].  Returns (codes float8_e4m3fn [..., D], scales float32 [..., D / block])."""
    _check(x.dtype == torch.bfloat16, "x must be bfloat16")
    _on_gpu(x)
    D = x.shape[-1]
    _check(D % block == 0, "the last dim must be a multiple of block")
    rows = x.numel() // D if D else 0
    codes = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scales = torch.empty((*x.shape[:-1], D // block), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().ks_fp8_quant_rows(_p(x), rows, D, block, 1 if ue8m0 else 0, _p(codes), _p(scales),
                                             _stream(x)), "fp8_quant")
    return codes, scales


def _fp8_codes(t: torch.Tensor) -> None:
    _check(t.dtype in (torch.float8_e4m3fn, torch.uint8), "codes must be float8_e4m3fn (or their uint8 bits)")


def indexer_fp8(q: torch.Tensor, q_scale: torch.Tensor, k: torch.Tensor, k_scale: torch.Tensor,
                weights: torch.Tensor, k_top: int, causal: bool, start_pos: int, ratio: int = 1, offset: int = 0,
                out_dtype: torch.dtype = torch.int32, workspace: Optional[torch.Tensor] = None,
                T: Optional[int] = None) -> torch.Tensor:
    """Indexer scores -> exact top-k on FP8 rows (as `indexer`, without RoPE: quantised rows are stored after
    it), with q_h = bf16(fp32(e4m3(q) * q_scale)) and k likewise, one scale per row.

    q: e4m3 [B, S, H, D], q_scale float32 [B, S, H]; k: e4m3 [B, Tk, D] with contiguous rows (batch-strided
    views accepted), k_scale float32 [B, Tk] with the same batch stride in rows; weights float32/bf16 [B, S, H].
    Returns [B, S, min(k_top, T)] int32 (default) or int64."""
    _fp8_codes(q)
    _fp8_codes(k)
    _check(q_scale.dtype == torch.float32 and k_scale.dtype == torch.float32, "scales must be float32")
    _check(weights.dtype in (torch.float32, torch.bfloat16), "weights must be float32 or bfloat16")
    _on_gpu(q, q_scale, weights)
    _on_gpu(k, k_scale, contiguous=False)
    _check(q.dim() == 4 and k.dim() == 3 and weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]")
    B, S, H, D = q.shape
    _check(k.shape[0] >= B and k.shape[2] == D, "k shape mismatch")
    _check(tuple(weights.shape) == (B, S, H) and tuple(q_scale.shape) == (B, S, H), "weights / q_scale shape")
    _check(q.is_contiguous() and q_scale.is_contiguous() and weights.is_contiguous(),
           "q, q_scale and weights must be contiguous")
    _check(k.stride(2) == 1 and k.stride(1) == D and k.stride(0) % D == 0, "k rows must be contiguous")
    _check(k_scale.dim() == 2 and k_scale.shape[0] >= B and k_scale.shape[1] == k.shape[1]
           and k_scale.stride(1) == 1, "k_scale [b, t] with contiguous rows")
    T = k.shape[1] if T is None else T
    _check(1 <= T <= k.shape[1], "T out of range")
    kbs = k.stride(0) // D if B > 1 else max(k.shape[1], T)
    _check(B <= 1 or k_scale.stride(0) == kbs, "k_scale must have the batch stride of k (in rows)")
    need = indexer_workspace_size(B, S, H, D, T)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    kk = min(k_top, T)
    out = torch.empty((B, S, kk), dtype=out_dtype, device=q.device)
    _lib.check(_lib.load().ks_indexer_fp8(_p(q), _p(q_scale), _p(k), _p(k_scale), _p(weights),
                                          1 if weights.dtype == torch.bfloat16 else 0, k_top, 1 if causal else 0,
                                          start_pos, ratio, offset, _p(out), 1 if out_dtype == torch.int64 else 0,
                                          B, S, H, D, T, kbs, _p(workspace), workspace.numel(), _stream(q)),
               "indexer_fp8")
    return out


# ---------------------------------------------------------------- sparse attention
@functools.lru_cache(maxsize=256)  # a pure function of the shape
def sparse_attn_workspace_size(B: int, M: int, H: int, Dqk: int, Dv: int, K: int) -> int:
    return int(_lib.load().ks_sparse_attn_workspace_size(B, M, H, Dqk, Dv, K))


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                softmax_scale: float, dv: Optional[int] = None,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sparse_attn_megakernel_basic(q, kv, attn_sink, topk_idxs, softmax_scale)
    (optimized/sparse_attention/op_extension/register.cpp:9-10), plus dv (V = kv[..., :dv]).

    q: bf16 [B, M, H, Dqk]; kv: bf16 [B, N, Dqk]; attn_sink: float32 [H]; topk_idxs: int32 [B, M, K]
    (negative = invalid).  Returns bf16 [B, M, H, dv]."""
    _check(q.dtype == torch.bfloat16, "q must be bfloat16")
    _check(kv.dtype == torch.bfloat16, "kv must be bfloat16")
    _check(attn_sink.dtype == torch.float32, "attn_sink must be float32")
    _check(topk_idxs.dtype == torch.int32, "topk_idxs must be int32")
    _on_gpu(q, kv, attn_sink, topk_idxs)
    _check(q.dim() == 4 and kv.dim() == 3 and attn_sink.dim() == 1 and topk_idxs.dim() == 3,
           "q [b,m,h,d], kv [b,n,d], attn_sink [h], topk_idxs [b,m,topk]")
    B, M, H, D = q.shape
    N = kv.shape[1]
    K = topk_idxs.shape[2]
    _check(kv.shape[0] == B and kv.shape[2] == D, "kv shape mismatch")
    _check(attn_sink.shape[0] == H, "attn_sink shape mismatch")
    _check(topk_idxs.shape[0] == B and topk_idxs.shape[1] == M, "topk_idxs shape mismatch")
    dv = D if dv is None else dv
    out = torch.empty((B, M, H, dv), dtype=torch.bfloat16, device=q.device)
    need = sparse_attn_workspace_size(B, M, H, D, dv, K)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    wsz = 0 if workspace is None else workspace.numel()
    _lib.check(_lib.load().ks_sparse_attn(_p(q), _p(kv), _p(attn_sink), _p(topk_idxs), _p(out), B, M, H, D, dv, N, K,
                                          float(softmax_scale), _p(workspace) if need else None, wsz, _stream(q)),
               "sparse_attn")
    return out


# ---------------------------------------------------------------- mHC hyper-connections
def _mhc_streams(x: torch.Tensor) -> None:
    _check(x.dtype == torch.bfloat16, "x must be bfloat16")
    _on_gpu(x)
    _check(x.dim() == 3 and x.shape[1] == 4 and x.shape[2] % 8 == 0, "x must be [N, 4, C] with C a multiple of 8")


def mhc_pre(x: torch.Tensor, pre_logits: torch.Tensor) -> torch.Tensor:
    """Layer input of an mHC block: h[t] = sum_j sigmoid(pre_logits[t, j]) x[t, j] (bf16 [N, C])."""
    _mhc_streams(x)
    _check(pre_logits.dtype == torch.float32 and tuple(pre_logits.shape) == (x.shape[0], 4),
           "pre_logits must be float32 [N, 4]")
    _on_gpu(pre_logits)
    N, _, C = x.shape
    h = torch.empty((N, C), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().ks_mhc_pre(_p(x), _p(pre_logits), _p(h), N, C, _stream(x)), "mhc_pre")
    return h


def mhc_post(x: torch.Tensor, f: torch.Tensor, res_logits: torch.Tensor, post_logits: torch.Tensor,
             sinkhorn_iters: int = 20, eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Residual update of an mHC block with the Sinkhorn fused in: out[t, i] = sum_j S(res_logits[t])[i, j] x[t, j]
    + 2 sigmoid(post_logits[t, i]) f[t], S = the Sinkhorn of sinkhorn() (repeat = sinkhorn_iters).  out may be x."""
    _mhc_streams(x)
    N, _, C = x.shape
    _check(f.dtype == torch.bfloat16 and tuple(f.shape) == (N, C), "f must be bfloat16 [N, C]")
    _check(res_logits.dtype == torch.float32 and tuple(res_logits.shape) == (N, 4, 4),
           "res_logits must be float32 [N, 4, 4]")
    _check(post_logits.dtype == torch.float32 and tuple(post_logits.shape) == (N, 4),
           "post_logits must be float32 [N, 4]")
    _on_gpu(f, res_logits, post_logits)
    if out is None:
        out = torch.empty_like(x)
    _check(out.dtype == torch.bfloat16 and out.shape == x.shape and out.is_contiguous(), "out must match x")
    _lib.check(_lib.load().ks_mhc_post(_p(x), _p(f), _p(res_logits), _p(post_logits), _p(out), N, C,
                                       int(sinkhorn_iters), float(eps), _stream(x)), "mhc_post")
    return out


def copy_bytes(src: torch.Tensor, dst: torch.Tensor) -> None:
    """Streaming copy kernel used to calibrate HBM traffic counters."""
    _on_gpu(src, dst)
    n = src.numel() * src.element_size()
    _check(dst.numel() * dst.element_size() >= n, "dst too small")
    _lib.check(_lib.load().ks_copy_bytes(_p(src), _p(dst), n, _stream(src)), "copy_bytes")
