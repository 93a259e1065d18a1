"""Torch-CPU restatement of the reference's baseline ops, op for op — TEST / BENCH ONLY.

This is the "host-CPU reference" that bench.py times on the GPU box's host cores
(cpu_baseline kind "port") and that tests use as a second, independent
floating-point check.  It issues the same torch op sequence as the reference's
frozen baselines (which never ship with this repository):

  sinkhorn      baseline/sinkhorn.py:13-19       softmax, +eps, colnorm, (row, col) x (repeat-1)
  indexer       baseline/indexer.py:114-129,161-206  complex RoPE, bf16 einsum, relu_, * w,
                                                  sum over heads, causal -inf, topk, -1/offset
  sparse_attn   baseline/sparse_attention.py:5-42 gather, fp32 einsum, sink softmax, fp32 einsum

The indexer here is generalised the same way as the HIP op (RoPE on a chosen
segment of q and optionally k, fp32 or bf16 head weights, causal at any start
position).  CPU torch.topk does not promise lowest-index-first ties, so exact
index comparisons use oracle.topk_stable instead; this module is for timing and
for tolerance-level cross-checks.
"""
from __future__ import annotations

import torch


def sinkhorn(x: torch.Tensor, repeat: int = 10, eps: float = 1e-6) -> torch.Tensor:
    y = x.softmax(-1) + eps
    y = y / (y.sum(-2, keepdim=True) + eps)
    for _ in range(repeat - 1):
        y = y / (y.sum(-1, keepdim=True) + eps)
        y = y / (y.sum(-2, keepdim=True) + eps)
    return y


def rope_(x: torch.Tensor, cis: torch.Tensor) -> torch.Tensor:
    """In-place complex rotation of x's last axis (pairs), bf16 in/out, fp32 math.

    x: [B, S, H, R] or [B, S, R] view; cis: complex64 [S, R/2]."""
    xc = torch.view_as_complex(x.float().unflatten(-1, (-1, 2)))
    if xc.ndim == 3:
        c = cis.view(1, xc.size(1), xc.size(-1))
    else:
        c = cis.view(1, xc.size(1), 1, xc.size(-1))
    x.copy_(torch.view_as_real(xc * c).flatten(-2))
    return x


def indexer_scores(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, cis: torch.Tensor, causal: bool,
                   start_pos: int, ratio: int = 1, rope_start: int = 0, rope_dim: int = 64,
                   rope_k: bool = True) -> torch.Tensor:
    """Scores [B, S, T] by the reference's op sequence: complex RoPE, bf16 einsum, relu_, * w, sum over
    heads, -inf mask (fp32 with fp32 weights, bf16 with bf16 weights, as torch computes them).

    q bf16 [B,S,H,D]; k bf16 [B,T,D]; w fp32 or bf16 [B,S,H]; cis complex64 [n_pos, rope_dim/2]."""
    B, S, H, D = q.shape
    T = k.shape[1]
    q = q.clone()
    k = k.clone()
    if rope_dim > 0:
        rope_(q[..., rope_start:rope_start + rope_dim], cis[start_pos:start_pos + S])
        if rope_k:
            rope_(k[..., rope_start:rope_start + rope_dim], cis[:T])
    score = torch.einsum("bshd,btd->bsht", q, k)
    score = (score.relu_() * w.unsqueeze(-1)).sum(dim=2)
    if causal:
        kpos = torch.arange(T).repeat(S, 1)
        lim = (start_pos + torch.arange(1, S + 1)).unsqueeze(1) // ratio
        score += torch.where(kpos >= lim, float("-inf"), 0.0)
    return score


def indexer(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, cis: torch.Tensor, k_top: int, causal: bool,
            start_pos: int, ratio: int = 1, offset: int = 0, rope_start: int = 0, rope_dim: int = 64,
            rope_k: bool = True) -> torch.Tensor:
    """q bf16 [B,S,H,D]; k bf16 [B,T,D]; w fp32 or bf16 [B,S,H]; cis complex64 [n_pos, rope_dim/2]."""
    S, T = q.shape[1], k.shape[1]
    score = indexer_scores(q, k, w, cis, causal, start_pos, ratio, rope_start, rope_dim, rope_k)
    kk = min(k_top, T)
    idx = score.topk(kk, dim=-1)[1]
    if causal:
        lim = (start_pos + torch.arange(1, S + 1)).unsqueeze(1) // ratio
        idx = torch.where(idx >= lim, -1, idx + offset)
    else:
        idx = idx + offset
    return idx


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, sink: torch.Tensor, idx: torch.Tensor, scale: float,
                dv: int | None = None) -> torch.Tensor:
    B, M, H, D = q.shape
    K = idx.shape[-1]
    ok = idx >= 0
    safe = idx.clamp_min(0).long()
    bi = torch.arange(B, device=idx.device)[:, None, None].expand(B, M, K)
    g = kv[bi, safe].masked_fill(~ok.unsqueeze(-1), 0.0)
    s = torch.einsum("bmhd,bmtd->bmht", q.float(), g.float()) * scale
    s = s.masked_fill(~ok.unsqueeze(2), float("-inf"))
    sk = sink.float().view(1, 1, H, 1)
    z = torch.maximum(torch.amax(s, dim=-1, keepdim=True), sk)
    e = torch.exp(s - z).masked_fill(~ok.unsqueeze(2), 0.0)
    p = e / (e.sum(dim=-1, keepdim=True) + torch.exp(sk - z))
    v = g if dv is None else g[..., :dv]
    return torch.einsum("bmht,bmtd->bmhd", p, v.float()).to(q.dtype)
