"""mHC residual hyper-connections (hc_mult = 4) on the fused gfx950 mixing kernels.

The reference configures manifold-constrained hyper-connections for its DeepSeek block (hc_mult = 4,
hc_sinkhorn_iters = 20, hc_eps = 1e-6; baseline/indexer.py:48-50) and ships their 4x4 Sinkhorn projection as
an operator of its own (baseline/sinkhorn.py).  HyperConnection keeps the four residual streams of a token,
x [N, 4, C], and computes per token, from the RMS-normalised flattened streams,
    logits = alpha * (x_norm @ phi) + base   ->  pre [4], post [4], res [4, 4];
the layer input h = sigmoid(pre) . x runs in ks_mhc_pre, and the residual update
    x' = Sinkhorn(res) x + 2 sigmoid(post) f(h)
in ks_mhc_post, whose kernel normalises each token's 4x4 logits in registers (the Sinkhorn of
torch.ops.ks_mi355x.sinkhorn, repeat = hc_sinkhorn_iters) and mixes the streams in the same pass.  The
logit projection stays a torch GEMM, as the reference keeps its projections in torch.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib


class HyperConnection(nn.Module):
    def __init__(self, dim: int, hc_mult: int = 4, hc_sinkhorn_iters: int = 20, hc_eps: float = 1e-6,
                 norm_eps: float = 1e-6):
        super().__init__()
        if hc_mult != 4:
            raise ValueError("the fused mixing kernels are built for hc_mult = 4")
        n = hc_mult
        self.dim, self.hc_mult = dim, n
        self.hc_sinkhorn_iters, self.hc_eps, self.norm_eps = hc_sinkhorn_iters, hc_eps, norm_eps
        self.phi = nn.Parameter(torch.randn(n * dim, 2 * n + n * n) * (n * dim) ** -0.5)
        self.alpha = nn.Parameter(torch.full((3,), 0.1))
        self.base = nn.Parameter(torch.zeros(2 * n + n * n))

    def logits(self, x: torch.Tensor):
        """(pre [N, 4], post [N, 4], res [N, 4, 4]) float32 from the streams x bf16 [N, 4, C]."""
        n = self.hc_mult
        xf = x.flatten(1).float()
        xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.norm_eps)
        z = xn @ self.phi
        pre = self.alpha[0] * z[:, :n] + self.base[:n]
        post = self.alpha[1] * z[:, n:2 * n] + self.base[n:2 * n]
        res = (self.alpha[2] * z[:, 2 * n:] + self.base[2 * n:]).view(-1, n, n)
        return pre.contiguous(), post.contiguous(), res.contiguous()

    def pre(self, x: torch.Tensor):
        """The layer input h bf16 [N, C] and the logits the residual update needs."""
        pre, post, res = self.logits(x)
        return _lib.torch_ops().mhc_pre(x, pre), post, res

    def post(self, x: torch.Tensor, f: torch.Tensor, post: torch.Tensor, res: torch.Tensor) -> torch.Tensor:
        """The next streams x' bf16 [N, 4, C] from the layer output f bf16 [N, C]."""
        return _lib.torch_ops().mhc_post(x, f, res, post, self.hc_sinkhorn_iters, self.hc_eps)

    def forward(self, x: torch.Tensor, layer) -> torch.Tensor:
        h, post, res = self.pre(x)
        return self.post(x, layer(h), post, res)
