"""The reference's baseline torch modules, restated — TEST INFRASTRUCTURE ONLY.

The drop-in check (tests/dropin_harness.py, tests/test_gpu_dropin.py) needs the "v0" side of the reference
harness: a Model with the baseline's constructor, parameter / buffer names and forward, from which the
harness copies the state dict into ModelNew and whose output it compares.  These classes restate
baseline/sinkhorn.py:5-19, baseline/indexer.py:132-206 and baseline/sparse_attention.py:45-65 op for op
(the same torch calls; oracle/torch_ref.py holds the shared functional forms), together with the
get_inputs / get_init_inputs example shapes of those files (baseline/indexer.py:53-64, 209-242;
baseline/sparse_attention.py:68-76; baseline/sinkhorn.py:22-29).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn

from oracle import torch_ref


class SinkhornModel(nn.Module):
    """baseline/sinkhorn.py:5-19."""

    def __init__(self, repeat: int = 10, eps: float = 1e-6):
        super().__init__()
        self.repeat = repeat
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch_ref.sinkhorn(x, self.repeat, self.eps)


def sinkhorn_get_inputs():
    return [torch.randn(1, 1024, 4, 4, dtype=torch.float32)]


def sinkhorn_get_init_inputs():
    return []


@dataclass
class IndexerArgs:
    """The ModelArgs fields the indexer reads, at the baseline's make_args() values (baseline/indexer.py:53-64)."""
    max_batch_size: int = 8
    max_seq_len: int = 2600
    dim: int = 1024
    index_n_heads: int = 16
    index_head_dim: int = 64
    index_topk: int = 128
    q_lora_rank: int = 256
    rope_head_dim: int = 32


def _linear(in_f: int, out_f: int) -> nn.Linear:
    lin = nn.Linear(in_f, out_f, bias=False, dtype=torch.bfloat16)
    nn.init.kaiming_uniform_(lin.weight, a=math.sqrt(5))
    return lin


class IndexerModel(nn.Module):
    """baseline/indexer.py:132-206: projections, RoPE on the last rope_head_dim dims of q, bf16 einsum against
    the (un-rotated) compressed cache, relu * weights summed over heads, causal mask and -1 post-processing
    only when start_pos == 0, +offset otherwise."""

    def __init__(self, args, freqs_cis: torch.Tensor, kv_cache: torch.Tensor, compress_ratio: int = 4):
        super().__init__()
        self.dim = args.dim
        self.n_heads = args.index_n_heads
        self.head_dim = args.index_head_dim
        self.rope_head_dim = args.rope_head_dim
        self.index_topk = args.index_topk
        self.wq_b = _linear(args.q_lora_rank, self.n_heads * self.head_dim)
        self.weights_proj = _linear(self.dim, self.n_heads)
        self.softmax_scale = self.head_dim ** -0.5
        self.compress_ratio = compress_ratio
        self.register_buffer("kv_cache", kv_cache)
        self.register_buffer("freqs_cis", freqs_cis)

    def scores(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int) -> torch.Tensor:
        bsz, seqlen, _ = x.size()
        ratio = self.compress_ratio
        end_pos = start_pos + seqlen
        q = self.wq_b(qr).unflatten(-1, (self.n_heads, self.head_dim))
        torch_ref.rope_(q[..., -self.rope_head_dim:], self.freqs_cis[start_pos:end_pos])
        weights = self.weights_proj(x) * (self.softmax_scale * self.n_heads ** -0.5)
        score = torch.einsum("bshd,btd->bsht", q, self.kv_cache[:bsz, :end_pos // ratio])
        score = (score.relu_() * weights.unsqueeze(-1)).sum(dim=2)
        if start_pos == 0:
            kpos = torch.arange(seqlen // ratio, device=x.device).repeat(seqlen, 1)
            lim = torch.arange(1, seqlen + 1, device=x.device).unsqueeze(1) // ratio
            score += torch.where(kpos >= lim, float("-inf"), 0.0)
        return score

    def forward(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int) -> torch.Tensor:
        seqlen = x.size(1)
        end_pos = start_pos + seqlen
        score = self.scores(x, qr, start_pos)
        idx = score.topk(min(self.index_topk, end_pos // self.compress_ratio), dim=-1)[1]
        if start_pos == 0:
            lim = torch.arange(1, seqlen + 1, device=x.device).unsqueeze(1) // self.compress_ratio
            idx = torch.where(idx >= lim, -1, idx + offset)
        else:
            idx += offset
        return idx


def indexer_get_inputs():
    a = IndexerArgs()
    x = torch.randn(a.max_batch_size, a.max_seq_len, a.dim, dtype=torch.bfloat16)
    qr = torch.randn(a.max_batch_size, a.max_seq_len, a.q_lora_rank, dtype=torch.bfloat16)
    return [x, qr, 0, 0]


def indexer_get_init_inputs():
    a = IndexerArgs()
    ratio = 4
    inv = 1.0 / (10000.0 ** (torch.arange(0, a.rope_head_dim, 2).float() / a.rope_head_dim))
    ang = torch.outer(torch.arange(a.max_seq_len, dtype=torch.float32), inv)
    freqs_cis = torch.polar(torch.ones_like(ang), ang)
    kv_cache = torch.randn(a.max_batch_size, a.max_seq_len // ratio, a.index_head_dim, dtype=torch.bfloat16)
    return [a, freqs_cis, kv_cache, ratio]


class SparseAttentionModel(nn.Module):
    """baseline/sparse_attention.py:45-65 (attn_sink parameter of zeros, softmax_scale = head_dim^-0.5)."""

    def __init__(self, n_heads: int, head_dim: int):
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.softmax_scale = head_dim ** -0.5
        self.attn_sink = nn.Parameter(torch.zeros(n_heads, dtype=torch.float32))

    def forward(self, q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        return torch_ref.sparse_attn(q, kv, self.attn_sink, topk_idxs, self.softmax_scale)


def sparse_get_inputs():
    q = torch.randn(8, 2600, 64, 128, dtype=torch.bfloat16)
    kv = torch.randn(8, 32, 128, dtype=torch.bfloat16)
    topk_idxs = torch.randint(0, 32, (8, 2600, 16), dtype=torch.int32)
    return [q, kv, topk_idxs]


def sparse_get_init_inputs():
    return [64, 128]
