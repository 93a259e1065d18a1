"""GPU parity of the mHC mixing kernels (the Sinkhorn fused into the residual update) against the fp64 oracle
(oracle.mhc_pre / oracle.mhc_post, whose Sinkhorn is oracle.sinkhorn): bf16 outputs within atol = rtol = 1e-2
(north star), and the fp32 arithmetic checked tighter against the oracle before its bf16 rounding."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import _lib, ops, workloads
from kernelswift_amd.mhc import HyperConnection

pytestmark = pytest.mark.gpu

bits = workloads.bf16_bits


def _inputs(g, N, C, scale=1.0):
    x = (torch.randn(N, 4, C, generator=g) * scale).bfloat16()
    f = torch.randn(N, C, generator=g).bfloat16()
    res = torch.randn(N, 4, 4, generator=g) * 2
    post = torch.randn(N, 4, generator=g)
    pre = torch.randn(N, 4, generator=g)
    return x, f, res, post, pre


def _close(got, want):
    # bf16 outputs: the north star's tolerance, and within two bf16 roundings of the fp64 value
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(got, want, atol=2 * 2.0 ** -8 * np.abs(want).max(), rtol=2.0 ** -7)


@pytest.mark.parametrize("N,C,iters", [(4096, 4096, 20), (37, 1032, 20), (5, 8, 1), (130, 7168, 10)])
def test_mhc_post_matches_oracle(device, N, C, iters):
    g = torch.Generator().manual_seed(N + C)
    x, f, res, post, _ = _inputs(g, N, C)
    print(f"[case] mhc_post N={N} C={C} iters={iters}", flush=True)
    out = ops.mhc_post(x.to(device), f.to(device), res.to(device), post.to(device), iters, 1e-6)
    got = out.float().cpu().numpy()
    rows = slice(0, min(N, 512))  # the fp64 oracle on a bounded sample of tokens at the large shape
    want = oracle.mhc_post(bits(x[rows]), bits(f[rows]), res[rows].numpy(), post[rows].numpy(), iters, 1e-6)
    _close(got[rows], want)


@pytest.mark.parametrize("N,C", [(4096, 4096), (37, 1032), (3, 8)])
def test_mhc_pre_matches_oracle(device, N, C):
    g = torch.Generator().manual_seed(N * 3 + C)
    x, _, _, _, pre = _inputs(g, N, C)
    print(f"[case] mhc_pre N={N} C={C}", flush=True)
    h = ops.mhc_pre(x.to(device), pre.to(device)).float().cpu().numpy()
    rows = slice(0, min(N, 512))
    _close(h[rows], oracle.mhc_pre(bits(x[rows]), pre[rows].numpy()))


def test_mhc_post_in_place_and_torch_op(device):
    g = torch.Generator().manual_seed(3)
    x, f, res, post, pre = _inputs(g, 64, 512)
    xd, fd, rd, pd = x.to(device), f.to(device), res.to(device), post.to(device)
    want = ops.mhc_post(xd, fd, rd, pd)
    t = _lib.torch_ops()
    assert torch.equal(t.mhc_post(xd, fd, rd, pd, 20, 1e-6), want)
    assert torch.equal(t.mhc_pre(xd, pre.to(device)), ops.mhc_pre(xd, pre.to(device)))
    xi = xd.clone()
    ops.mhc_post(xi, fd, rd, pd, out=xi)  # the update may overwrite its own streams
    assert torch.equal(xi, want)


def test_mhc_post_sinkhorn_is_the_fused_one(device):
    # with x = identity-like streams (stream j = e_j pattern) the mixed output exposes the matrix itself:
    # out[t, i, j] = S[t, i, j] for C = 8 with x[t, j, c] = [c == j] and the layer output switched off
    g = torch.Generator().manual_seed(4)
    N = 256
    x = torch.zeros(N, 4, 8)
    for j in range(4):
        x[:, j, j] = 1.0
    res = torch.randn(N, 4, 4, generator=g) * 3
    post = torch.full((N, 4), -200.0)
    out = ops.mhc_post(x.bfloat16().to(device), torch.zeros(N, 8).bfloat16().to(device), res.to(device),
                       post.to(device), 20, 1e-6).float().cpu().numpy()
    S = ops.sinkhorn(res.to(device), 20, 1e-6).cpu().numpy()
    np.testing.assert_allclose(out[:, :, :4], S, atol=2.0 ** -8, rtol=2.0 ** -8)  # bf16 rounding of S
    np.testing.assert_allclose(S, oracle.sinkhorn(res.numpy(), 20, 1e-6), atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(S.sum(-2), 1.0, atol=1e-4)  # the last pass normalises the columns


def test_hyper_connection_layer(device):
    # the layer end to end (torch projection for the logits, then the two fused kernels) against an fp64
    # restatement on the module's own logits
    torch.manual_seed(7)
    hc = HyperConnection(dim=1024).to(device)
    x = torch.randn(96, 4, 1024).bfloat16().to(device)
    w = (torch.randn(1024, 1024) * 0.03).bfloat16().to(device)
    layer = lambda h: h @ w  # noqa: E731
    with torch.no_grad():
        out = hc(x, layer)
        pre, post, res = hc.logits(x)
        h = ops.mhc_pre(x, pre)
        fo = layer(h)
    want_h = oracle.mhc_pre(bits(x), pre.cpu().numpy())
    _close(h.float().cpu().numpy(), want_h)
    want = oracle.mhc_post(bits(x), bits(fo), res.cpu().numpy(), post.cpu().numpy(), 20, 1e-6)
    _close(out.float().cpu().numpy(), want)
