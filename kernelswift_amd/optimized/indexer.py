"""Indexer drop-in: ModelNew(args, freqs_cis, kv_cache, compress_ratio=4).forward(x, qr, start_pos, offset).

Constructor, forward signature, parameter names (wq_b.weight, weights_proj.weight) and buffers (kv_cache,
freqs_cis) of the reference indexer (baseline/indexer.py:132-206; optimized/indexer_project/indexer.py:
168-224), so a state dict of the baseline Model loads as is.  The two projections stay torch GEMMs, as in
the reference; RoPE of q (last rope_head_dim dims), the exact score contraction with the ReLU * weight head
reduction and the causal mask, and the exact sorted top-k with the -1 / +offset post-processing run as one
call of the fused gfx950 operator torch.ops.ks_mi355x.indexer (ks_indexer), without a transposed or padded copy
of the cache.

Semantics kept from the baseline: weights = weights_proj(x) * (head_dim^-0.5 * n_heads^-0.5) in bf16 (the product
is taken inside the fused call, w_scale, with torch's rounding: no separate multiply launch);
keys are kv_cache[:B, :(start_pos + S) // ratio] (not rotated); the causal mask and the -1 post-processing
apply only when start_pos == 0; output int64 [B, S, min(index_topk, (start_pos + S) // ratio)].  Scores
follow the exact canonical arithmetic of include/kswift.h, and ties keep the lowest key index first.
"""
import os
import sys
from dataclasses import dataclass

import torch
import torch.nn as nn


_OPS = None


def _ops():
    """torch.ops.ks_mi355x (libkswift_torch.so), loaded on first use like the reference wrappers' extension, then
    kept (a forward's first call into the library should not pay an import lookup)."""
    global _OPS
    if _OPS is None:
        root = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
        if root not in sys.path:
            sys.path.insert(0, root)
        from kernelswift_amd import _lib
        _OPS = _lib.torch_ops()
    return _OPS


@dataclass
class ModelArgs:
    """The fields of the reference ModelArgs (baseline/indexer.py:10-51) that the indexer reads; any object
    with these attributes (the reference's own ModelArgs included) is accepted."""
    max_batch_size: int = 4
    max_seq_len: int = 4096
    dim: int = 4096
    index_n_heads: int = 64
    index_head_dim: int = 128
    index_topk: int = 512
    q_lora_rank: int = 1024
    rope_head_dim: int = 64


class ModelNew(nn.Module):
    def __init__(self, args, freqs_cis: torch.Tensor, kv_cache: torch.Tensor, compress_ratio: int = 4):
        super().__init__()
        self.dim = args.dim
        self.n_heads = args.index_n_heads
        self.n_local_heads = args.index_n_heads
        self.head_dim = args.index_head_dim
        self.rope_head_dim = args.rope_head_dim
        self.index_topk = args.index_topk
        self.q_lora_rank = args.q_lora_rank
        self.wq_b = nn.Linear(self.q_lora_rank, self.n_heads * self.head_dim, bias=False, dtype=torch.bfloat16)
        self.weights_proj = nn.Linear(self.dim, self.n_heads, bias=False, dtype=torch.bfloat16)
        self.softmax_scale = self.head_dim ** -0.5
        self.compress_ratio = compress_ratio
        self.register_buffer("kv_cache", kv_cache)
        self.register_buffer("freqs_cis", freqs_cis)
        self._freqs_key = None
        self._freqs_val = None

    def _freqs(self) -> torch.Tensor:
        """(cos, sin) float32 [rows, rope_head_dim/2, 2] from the complex table (or its real view); kept between
        calls while the buffer (storage, version, dtype, shape) is unchanged."""
        f = self.freqs_cis
        key = (f.data_ptr(), f._version, f.dtype, tuple(f.shape), f.device)
        if key != self._freqs_key:
            g = torch.view_as_real(f) if f.is_complex() else f
            self._freqs_val = g.reshape(g.shape[0], -1, 2).to(torch.float32).contiguous()
            self._freqs_key = key
        return self._freqs_val

    def forward(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int) -> torch.Tensor:
        ops = _ops()
        bsz, seqlen, _ = x.size()
        ratio = self.compress_ratio
        end_pos = start_pos + seqlen
        T = end_pos // ratio
        k_top = min(self.index_topk, T)
        if k_top == 0:
            return torch.empty((bsz, seqlen, 0), dtype=torch.int64, device=x.device)
        q = self.wq_b(qr).unflatten(-1, (self.n_local_heads, self.head_dim)).contiguous()
        weights = self.weights_proj(x).contiguous()
        return ops.indexer(q, self.kv_cache[:bsz], weights, self._freqs(), k_top, start_pos == 0, start_pos, ratio,
                           offset, self.head_dim - self.rope_head_dim, self.rope_head_dim, False, True, T,
                           w_scale=self.softmax_scale * self.n_heads ** -0.5)


def _example_args() -> ModelArgs:
    return ModelArgs(max_batch_size=8, max_seq_len=2600, dim=1024, index_n_heads=16, index_head_dim=64,
                     index_topk=128, q_lora_rank=256, rope_head_dim=32)


def get_inputs():
    args = _example_args()
    x = torch.randn(8, 2600, args.dim, dtype=torch.bfloat16)
    qr = torch.randn(8, 2600, args.q_lora_rank, dtype=torch.bfloat16)
    return [x, qr, 0, 0]


def get_init_inputs():
    args = _example_args()
    ratio = 4
    inv = 1.0 / (10000.0 ** (torch.arange(0, args.rope_head_dim, 2).float() / args.rope_head_dim))
    angles = torch.outer(torch.arange(args.max_seq_len, dtype=torch.float32), inv)
    freqs_cis = torch.polar(torch.ones_like(angles), angles)
    kv_cache = torch.randn(args.max_batch_size, args.max_seq_len // ratio, args.index_head_dim,
                           dtype=torch.bfloat16)
    return [args, freqs_cis, kv_cache, ratio]
