"""GPU parity: sparse attention kernel vs the fp64 oracle (atol = rtol = 1e-2, the reference contract
of benchmarks/ks/auto_bench.py:41-43), at configs 3 and 5, the reference's own example shape, and edge
cases: invalid (-1 / out-of-range) indices, duplicates, all-invalid rows, nonzero sinks."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu
bits = workloads.bf16_bits
TOL = dict(atol=1e-2, rtol=1e-2)


def _run(q, kv, sink, idx, scale, dv, tag):
    print(f"[case] sparse_attn {tag} q={tuple(q.shape)} kv={tuple(kv.shape)} K={idx.shape[-1]} dv={dv}", flush=True)
    out = ops.sparse_attn(q, kv, sink, idx, scale, dv=dv)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_sparse_attn_config3(device):
    w = workloads.CONFIGS[3]("cpu")
    t, p = w.tensors, w.params
    d = {n: v.to(device) for n, v in t.items()}
    got = _run(d["q"], d["kv"], d["sink"], d["idx"], p["scale"], p["dv"], "config3")
    want = oracle.sparse_attn(bits(t["q"]), bits(t["kv"]), t["sink"].numpy(), t["idx"].numpy(), p["scale"], p["dv"])
    np.testing.assert_allclose(got, want, **TOL)
    print(f"[info] config3 max abs diff {np.max(np.abs(got - want)):.3e}", flush=True)


def test_sparse_attn_config5(device):
    w = workloads.CONFIGS[5](device)
    t, p = w.tensors, w.params
    got = _run(t["q"], t["kv"], t["sink"], t["idx"], p["scale"], p["dv"], "config5")
    # oracle on the gathered rows only (the 2.25 GiB cache never leaves the GPU)
    B, _, K = t["idx"].shape
    rows = torch.stack([t["kv"][b, t["idx"][b, 0].long()] for b in range(B)])  # [B, K, 576]
    local = torch.arange(K, dtype=torch.int32).expand(B, 1, K).contiguous()
    want = oracle.sparse_attn(bits(t["q"]), bits(rows), t["sink"].cpu().numpy(), local.numpy(), p["scale"], p["dv"])
    np.testing.assert_allclose(got, want, **TOL)
    print(f"[info] config5 max abs diff {np.max(np.abs(got - want)):.3e}", flush=True)


def test_sparse_attn_reference_example_shape(device):
    # baseline/sparse_attention.py:101-117: B=8, H=64, N=32, D=128, topk=16 (randint -> duplicates);
    # M reduced from 2600 to 650 to keep the fp64 oracle fast
    g = torch.Generator().manual_seed(42)
    q = torch.randn(8, 650, 64, 128, generator=g).bfloat16()
    kv = torch.randn(8, 32, 128, generator=g).bfloat16()
    idx = torch.randint(0, 32, (8, 650, 16), generator=g, dtype=torch.int32)
    sink = torch.zeros(64)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), 128 ** -0.5, 128, "reference-example")
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx.numpy(), 128 ** -0.5, 128)
    np.testing.assert_allclose(got, want, **TOL)


@pytest.mark.parametrize("Dqk,Dv,H", [(128, 128, 16), (128, 128, 64), (576, 512, 128), (576, 512, 32),
                                      (576, 512, 48)])
def test_sparse_attn_edges(device, Dqk, Dv, H):
    g = torch.Generator().manual_seed(Dqk + H)
    B, M, N, K = 2, 5, 300, 100
    q = torch.randn(B, M, H, Dqk, generator=g).bfloat16()
    kv = torch.randn(B, N, Dqk, generator=g).bfloat16()
    idx = torch.randint(-20, N + 20, (B, M, K), generator=g, dtype=torch.int32)  # invalid: <0 and >=N
    idx[0, 0] = -1  # an all-invalid row -> output 0
    idx[0, 1, :50] = 7  # duplicates count with multiplicity
    sink = torch.randn(H, generator=g)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), Dqk ** -0.5, Dv, "edges")
    ok = (idx >= 0) & (idx < N)
    idx_o = torch.where(ok, idx, torch.full_like(idx, -1))
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx_o.numpy(), Dqk ** -0.5, Dv)
    np.testing.assert_allclose(got, want, **TOL)
    assert np.all(got[0, 0] == 0)


@pytest.mark.parametrize("K", [1, 31, 33, 2048, 4000])
def test_sparse_attn_split_counts(device, K):
    g = torch.Generator().manual_seed(K)
    B, M, H, N = 1, 3, 16, 5000
    q = torch.randn(B, M, H, 128, generator=g).bfloat16()
    kv = torch.randn(B, N, 128, generator=g).bfloat16()
    idx = torch.randint(0, N, (B, M, K), generator=g, dtype=torch.int32)
    sink = torch.full((H,), 0.5)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), 0.3, 128, f"K={K}")
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx.numpy(), 0.3, 128)
    np.testing.assert_allclose(got, want, **TOL)


# Small kv sets (N <= 64, Dqk = Dv = 128, H in {16, 32, 64}, K <= 256) take the dense count-mask kernel: duplicates
# count with multiplicity, indices < 0 or >= N count nowhere, an all-invalid row gives 0.  Every (N, K) tier and head
# count; M not a multiple of the queries a workgroup step covers (idle waves at each batch's end); batch boundaries
# inside a workgroup's range (restaging the kv rows); a single key; K above N (many duplicates).
@pytest.mark.parametrize("H,B,M,N,K", [(64, 2, 5, 32, 16), (16, 3, 7, 20, 40), (32, 2, 9, 64, 256), (16, 2, 3, 1, 1),
                                       (64, 3, 33, 48, 100), (32, 4, 130, 32, 64), (16, 1, 4097, 17, 65),
                                       (64, 8, 301, 32, 16)])
def test_sparse_attn_dense_small_kv(device, H, B, M, N, K):
    g = torch.Generator().manual_seed(H * 31 + N * 7 + K)
    q = torch.randn(B, M, H, 128, generator=g).bfloat16()
    kv = torch.randn(B, N, 128, generator=g).bfloat16()
    idx = torch.randint(-2, N + 2, (B, M, K), generator=g, dtype=torch.int32)  # invalid: < 0 and >= N
    idx[0, 0] = -1  # an all-invalid row -> output 0
    if M > 1:
        idx[0, 1, : (K + 1) // 2] = 0  # duplicates count with multiplicity
    sink = torch.randn(H, generator=g)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), 128 ** -0.5, 128,
               f"dense H={H} B={B} M={M} N={N} K={K}")
    ok = (idx >= 0) & (idx < N)
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), torch.where(ok, idx, -1).numpy(), 128 ** -0.5, 128)
    np.testing.assert_allclose(got, want, **TOL)
    assert np.all(got[0, 0] == 0)


def test_sparse_attn_errors(device):
    q = torch.zeros(1, 1, 16, 64, dtype=torch.bfloat16, device=device)
    kv = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=device)
    idx = torch.zeros(1, 1, 4, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError):
        ops.sparse_attn(q, kv, torch.zeros(16, device=device), idx, 0.1)  # D=64 unsupported
    with pytest.raises(RuntimeError):
        ops.sparse_attn(q.float(), kv, torch.zeros(16, device=device), idx, 0.1)


# MLA-shaped heads (Dqk 576, Dv 512, H a multiple of 32) run the 32-heads-per-wave kernel: one range per query
# (B*M >= 256, finalised in the kernel), split ranges with the combine, ranges capped at 2048 keys (K = 2049,
# 4000), ragged chunks (K = 1, 33), every wave count (H = 32, 64, 96, 128)
@pytest.mark.parametrize("H,B,M,K", [(32, 1, 256, 40), (64, 2, 3, 300), (96, 1, 2, 2049), (128, 2, 2, 4000),
                                     (128, 3, 1, 1), (128, 1, 1, 33)])
def test_sparse_attn_mla_shapes(device, H, B, M, K):
    g = torch.Generator().manual_seed(H * 7 + K)
    N = 3000
    q = torch.randn(B, M, H, 576, generator=g).bfloat16()
    kv = torch.randn(B, N, 576, generator=g).bfloat16()
    idx = torch.randint(-3, N, (B, M, K), generator=g, dtype=torch.int32)  # a few invalid (-1..-3)
    sink = torch.randn(H, generator=g)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), 576 ** -0.5, 512, f"mla H={H} K={K}")
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx.numpy(), 576 ** -0.5, 512)
    np.testing.assert_allclose(got, want, **TOL)


def _rising_case(g, H, K, jumps):
    """Scores equal up to small noise, except keys at positions `jumps` whose scores exceed the running maximum
    by ~9-13.5 (log2 units): each forces the online softmax to move its reference and rescale the accumulated
    O by 2^-9 or less, while the ~(position) earlier keys keep a total weight comparable to the new one."""
    N = 4096
    u = torch.randn(576, generator=g)
    scale = 576 ** -0.5
    base = 0.5 * u + 0.05 * torch.randn(N, 576, generator=g)
    step = 9.0 / (float(u @ u) * scale * 1.4426950408889634)  # +9 log2 units per jump at c = 1
    pos = torch.randperm(N, generator=g)[:K].to(torch.int32)
    for n, j in enumerate(jumps):
        base[int(pos[j])] = (0.5 + (n + 1) * step) * u
    c = 0.9 + 0.6 * torch.rand(H, generator=g)  # per-head gain: jumps of 8.1 .. 13.5
    q = (c[:, None] * u[None, :]).expand(1, 1, H, 576).contiguous().bfloat16()
    return q, base.unsqueeze(0).bfloat16(), pos.view(1, 1, K), scale


@pytest.mark.parametrize("H,jumps", [(128, [300]), (64, [300]), (32, [300]), (128, [40, 200, 330, 470])])
def test_sparse_attn_mla_rescale(device, H, jumps):
    g = torch.Generator().manual_seed(11 + H)
    K = 512
    q, kv, idx, scale = _rising_case(g, H, K, jumps)
    sink = torch.zeros(H)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), scale, 512, f"mla-rescale H={H}")
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx.numpy(), scale, 512)
    np.testing.assert_allclose(got, want, **TOL)
    if len(jumps) == 1:  # the ~500 earlier keys keep a weight comparable to the jump key's
        top = oracle.bf16_to_f32(bits(kv)[0, int(idx[0, 0, jumps[0]])])[:512]
        assert np.max(np.abs(want[0, 0] - top[None, :])) > 0.1


def test_sparse_attn_mla_leading_invalid(device):
    # the first chunks of every range are invalid: the references start at -inf without an O rescale
    g = torch.Generator().manual_seed(5)
    B, M, H, N, K = 1, 4, 128, 2000, 256
    q = torch.randn(B, M, H, 576, generator=g).bfloat16()
    kv = torch.randn(B, N, 576, generator=g).bfloat16()
    idx = torch.randint(0, N, (B, M, K), generator=g, dtype=torch.int32)
    idx[:, :, :100] = -1
    sink = torch.randn(H, generator=g)
    got = _run(q.to(device), kv.to(device), sink.to(device), idx.to(device), 576 ** -0.5, 512, "mla-leading-invalid")
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), idx.numpy(), 576 ** -0.5, 512)
    np.testing.assert_allclose(got, want, **TOL)


# The count-mask kernel (ks_dbg_sparse_attn_count: the dense formulation over key splits, timed beside the gather
# kernel by bench.py; ks_sparse_attn does not dispatch to it): one split finalised in place or several merged by the
# combine kernel; N not a multiple of the 32-key chunk; the last 128-row block of a batch partly past the batch;
# every head count; K above N (many duplicates); K not a multiple of 4 (the scalar count path); invalid indices on
# both sides; an all-invalid row; config 3's shape.
def _run_count(q, kv, sink, idx, scale, tag):
    print(f"[case] sparse_attn_count {tag}", flush=True)
    B, M, H, _ = q.shape
    N, K = kv.shape[1], idx.shape[-1]
    lib = _lib.load()
    need = lib.ks_sparse_attn_workspace_size(B, M, H, 128, 128, K)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    out = torch.empty(B, M, H, 128, dtype=torch.bfloat16, device=q.device)
    rc = lib.ks_dbg_sparse_attn_count(q.data_ptr(), kv.data_ptr(), sink.data_ptr(), idx.data_ptr(), out.data_ptr(), B, M,
                                      H, N, K, scale, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ks_dbg_sparse_attn_count")
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("H,B,M,N,K", [(16, 2, 9, 300, 100), (32, 1, 40, 1000, 600), (64, 2, 6, 2500, 1000),
                                       (128, 1, 3, 4100, 1200), (64, 1, 521, 200, 64), (16, 1, 16, 100, 300),
                                       (16, 1, 16, 100, 301), (16, 3, 24, 4096, 1024), (16, 1, 128, 8192, 2048)])
def test_sparse_attn_count_mask(device, H, B, M, N, K):
    g = torch.Generator().manual_seed(H * 13 + N + K)
    q = torch.randn(B, M, H, 128, generator=g).bfloat16()
    kv = torch.randn(B, N, 128, generator=g).bfloat16()
    idx = torch.randint(-3, N + 3, (B, M, K), generator=g, dtype=torch.int32)  # invalid: < 0 and >= N
    idx[0, 0] = -1  # an all-invalid row -> output 0
    idx[-1, -1, : K // 3] = N - 1  # duplicates count with multiplicity (the last key of the last split)
    sink = torch.randn(H, generator=g)
    got = _run_count(q.to(device), kv.to(device), sink.to(device), idx.to(device), 128 ** -0.5,
                     f"H={H} B={B} M={M} N={N} K={K}")
    ok = (idx >= 0) & (idx < N)
    want = oracle.sparse_attn(bits(q), bits(kv), sink.numpy(), torch.where(ok, idx, -1).numpy(), 128 ** -0.5, 128)
    np.testing.assert_allclose(got, want, **TOL)
    assert np.all(got[0, 0] == 0)
