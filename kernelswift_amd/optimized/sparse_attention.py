"""Sparse-attention drop-in: ModelNew(n_heads, head_dim).forward(q, kv, topk_idxs).

Signature and parameters of optimized/sparse_attention/sparse_attention.py:31-44 over
baseline/sparse_attention.py:45-65 (attn_sink parameter, softmax_scale = head_dim ** -0.5).  Gather, QK,
sink softmax and PV run in the gfx950 kernels behind torch.ops.ks_mi355x.sparse_attn (ks_sparse_attn).
q: bf16 [B, M, H, D]; kv: bf16 [B, N, D]; topk_idxs: int32 (or int64) [B, M, K], -1 = invalid.  Indices
outside [0, N) are invalid (masked, as the kernel treats them); int64 values are mapped to -1 before they
are narrowed to int32, so no out-of-range value can wrap onto a valid row.
"""
import os
import sys

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


class ModelNew(nn.Module):
    def __init__(self, n_heads: int, head_dim: int):
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.softmax_scale = head_dim ** -0.5
        self.attn_sink = nn.Parameter(torch.zeros(n_heads, dtype=torch.float32))

    def forward(self, q: torch.Tensor, kv: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        idx = topk_idxs
        if idx.dtype != torch.int32:
            idx = torch.where((idx < 0) | (idx >= kv.shape[1]), -1, idx).to(torch.int32)
        sink = self.attn_sink.detach()
        if sink.dtype != torch.float32:
            sink = sink.float()
        return _ops().sparse_attn(q.contiguous(), kv.contiguous(), sink.contiguous(), idx.contiguous(),
                                  self.softmax_scale)


def get_inputs():
    q = torch.randn(8, 2600, 64, 128, dtype=torch.bfloat16)
    kv = torch.randn(8, 32, 128, dtype=torch.bfloat16)
    topk_idxs = torch.randint(0, 32, (8, 2600, 16), dtype=torch.int32)
    return [q, kv, topk_idxs]


def get_init_inputs():
    return [64, 128]
