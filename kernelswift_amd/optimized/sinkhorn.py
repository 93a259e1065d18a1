"""Sinkhorn drop-in: ModelNew(repeat=10, eps=1e-6).forward(x).

Signature of optimized/sinkhorn_project/sinkhorn.py:35-52 over baseline/sinkhorn.py:5-19; the whole
normalisation (softmax + eps, then `repeat` row/column passes) is one gfx950 kernel behind the torch operator
torch.ops.ks_mi355x.sinkhorn (ks_sinkhorn).
x: float32 [..., 4, 4] on the GPU; returns a new float32 tensor of the same shape.
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
    def __init__(self, repeat: int = 10, eps: float = 1e-6):
        super().__init__()
        self.repeat = repeat
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _ops().sinkhorn(x.contiguous(), self.repeat, self.eps)


def get_inputs():
    return [torch.randn(1, 1024, 4, 4, dtype=torch.float32)]


def get_init_inputs():
    return []
