"""GPU parity of the drop-in ModelNew modules at the reference's own example shapes.

The reference harness builds ModelNew(*get_init_inputs()), loads the baseline Model's state dict and calls
forward(*get_inputs()) (benchmarks/ks/auto_bench.py:358-445, 505-533).  Here each ModelNew runs at the
example shapes of baseline/*.py and is checked against the CPU oracle: indices bit-exact (the projections
are the module's own torch GEMMs, evaluated once on the GPU and fed to the oracle), floating-point
outputs within atol = rtol = 1e-2."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import workloads
from kernelswift_amd.optimized import indexer as ix
from kernelswift_amd.optimized import sinkhorn as sk
from kernelswift_amd.optimized import sparse_attention as sa

pytestmark = pytest.mark.gpu

bits = workloads.bf16_bits


def test_sinkhorn_modelnew_example(device):
    torch.manual_seed(42)
    m = sk.ModelNew(*sk.get_init_inputs()).to(device)
    (x,) = sk.get_inputs()
    print("[case] sinkhorn ModelNew [1,1024,4,4]", flush=True)
    with torch.no_grad():
        y = m(x.to(device)).cpu().numpy()
    want = oracle.sinkhorn(x.numpy(), 10, 1e-6)
    np.testing.assert_allclose(y, want, atol=1e-2, rtol=1e-2)
    assert y.shape == (1, 1024, 4, 4)


def test_sparse_attention_modelnew_example(device):
    torch.manual_seed(42)
    m = sa.ModelNew(*sa.get_init_inputs()).to(device)
    with torch.no_grad():
        m.attn_sink.copy_(torch.linspace(-1, 1, 64))  # a non-trivial sink, as a loaded state dict may carry
    q, kv, idx = sa.get_inputs()
    idx[0, :5, :3] = -1  # invalid entries
    idx[1, 7, :] = 3     # duplicates
    print("[case] sparse_attention ModelNew [8,2600,64,128] N=32 K=16", flush=True)
    with torch.no_grad():
        out = m(q.to(device), kv.to(device), idx.to(device))
    got = out.float().cpu().numpy()
    want = oracle.sparse_attn(bits(q), bits(kv), m.attn_sink.detach().cpu().numpy(), idx.numpy(), 128 ** -0.5)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    assert out.dtype == torch.bfloat16 and out.shape == (8, 2600, 64, 128)


def _indexer_oracle(m, x, qr, start_pos, offset):
    with torch.no_grad():
        q = m.wq_b(qr).unflatten(-1, (m.n_heads, m.head_dim)).contiguous()
        w = m.weights_proj(x) * (m.softmax_scale * m.n_heads ** -0.5)
    B, S = x.shape[:2]
    T = (start_pos + S) // m.compress_ratio
    k = m.kv_cache[:B, :T].contiguous()
    freqs = torch.view_as_real(m.freqs_cis).cpu().numpy()
    return oracle.indexer(bits(q.cpu()), bits(k.cpu()), bits(w.cpu()), freqs, min(m.index_topk, T),
                          start_pos == 0, start_pos, m.compress_ratio, offset, m.head_dim - m.rope_head_dim,
                          m.rope_head_dim, False)


def test_indexer_modelnew_example_prefill(device):
    torch.manual_seed(42)
    m = ix.ModelNew(*ix.get_init_inputs()).to(device)
    x, qr, start_pos, offset = ix.get_inputs()
    x, qr = x.to(device), qr.to(device)
    print("[case] indexer ModelNew example B=8 S=2600 H=16 D=64 ratio=4 k=128 start_pos=0", flush=True)
    with torch.no_grad():
        got = m(x, qr, start_pos, offset)
    assert got.dtype == torch.int64 and got.shape == (8, 2600, 128)
    want = _indexer_oracle(m, x, qr, start_pos, offset)
    g = got.cpu().numpy()
    assert int((g != want).sum()) == 0
    # the first queries see fewer keys than k: their tails are -1
    assert (g[:, 0, :] == -1).all() and (g[:, 2599, :] >= 0).all()


@pytest.mark.parametrize("start_pos,offset", [(2000, 7), (3, 0)])
def test_indexer_modelnew_decode_offsets(device, start_pos, offset):
    torch.manual_seed(3)
    args = ix.ModelArgs(max_batch_size=4, max_seq_len=2600, dim=256, index_n_heads=32, index_head_dim=128,
                        index_topk=128, q_lora_rank=128, rope_head_dim=64)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    ang = torch.outer(torch.arange(2600, dtype=torch.float32), inv)
    m = ix.ModelNew(args, torch.polar(torch.ones_like(ang), ang), torch.randn(4, 650, 128).bfloat16(), 4).to(device)
    B, S = 3, 40
    x = torch.randn(B, S, 256).bfloat16().to(device)
    qr = torch.randn(B, S, 128).bfloat16().to(device)
    print(f"[case] indexer ModelNew start_pos={start_pos} offset={offset} H=32 D=128", flush=True)
    with torch.no_grad():
        got = m(x, qr, start_pos, offset)
    want = _indexer_oracle(m, x, qr, start_pos, offset)
    assert got.shape == want.shape
    assert int((got.cpu().numpy() != want).sum()) == 0
