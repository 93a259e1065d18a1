"""GPU: the indexer's top-k output feeds sparse attention directly on the device (int32 indices, -1 for
masked slots), the chaining of baseline/indexer.py:195-206 into baseline/sparse_attention.py:16-22.

The indices are compared bit for bit with the oracle's, and the attention output with the fp64 oracle run
on the oracle's indices (atol = rtol = 1e-2)."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import ops, workloads

pytestmark = pytest.mark.gpu

bits = workloads.bf16_bits


@pytest.mark.parametrize("start_pos,k_top", [(0, 64), (300, 128)])
def test_indexer_into_sparse_attn(device, start_pos, k_top):
    g = torch.Generator().manual_seed(start_pos + k_top)
    B, S, H, D, Ha = 2, 24, 64, 128, 16
    T = start_pos + S  # causal: query s sees keys t < start_pos + s + 1
    q_idx = torch.randn(B, S, H, D, generator=g).bfloat16()
    kv = torch.randn(B, T, D, generator=g).bfloat16()
    w = torch.randn(B, S, H, generator=g) / 8
    tab = workloads.freqs_table(64, 1024)
    q_att = torch.randn(B, S, Ha, D, generator=g).bfloat16()
    sink = torch.randn(Ha, generator=g)
    print(f"[case] chain start_pos={start_pos} k_top={k_top}", flush=True)
    kv_d = kv.to(device)
    idx = ops.indexer(q_idx.to(device), kv_d, w.to(device), tab.to(device), k_top, True, start_pos, 1, 0, 0, 64,
                      True)
    out = ops.sparse_attn(q_att.to(device), kv_d, sink.to(device), idx, D ** -0.5)
    torch.cuda.synchronize()
    want_idx = oracle.indexer(bits(q_idx), bits(kv), w.numpy(), tab.numpy(), k_top, True, start_pos, 1, 0, 0, 64,
                              True)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), want_idx)
    assert (want_idx < 0).any() == (start_pos + 1 < min(k_top, T))  # early queries have masked slots
    want = oracle.sparse_attn(bits(q_att), bits(kv), sink.numpy(), want_idx.astype(np.int32), D ** -0.5)
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("start_pos,offset", [(0, 128), (1200, 64)])
def test_compressed_indexer_into_mla_sparse_attn(device, start_pos, offset):
    # The DeepSeek-style chain at the row's named formats: the indexer scores S queries against a compressed
    # index cache [B, T/4, 128] (compress ratio 4; query s sees compressed keys t < (start_pos + s + 1) / 4),
    # and its int32 output (-1 where masked, else t + offset) indexes an MLA latent cache [B, offset + T/4,
    # 576] whose first `offset` rows stand for the uncompressed window: sparse attention with Dqk 576 / Dv
    # 512 (V = the 512 latent dims) and 64 heads, all on the device.  (baseline/indexer.py:179, 195-206,
    # 236-241 into baseline/sparse_attention.py:16-22.)
    g = torch.Generator().manual_seed(start_pos + offset)
    B, S, H, D, ratio, k_top = 2, 64, 64, 128, 4, 96
    T = (start_pos + S) // ratio  # compressed keys visible to the last query
    Ha, Dqk, Dv = 64, 576, 512
    q_idx = torch.randn(B, S, H, D, generator=g).bfloat16()
    kcache = torch.randn(B, T + 5, D, generator=g).bfloat16()  # rows past T exist in the cache, unused
    w = torch.randn(B, S, H, generator=g) / 8
    tab = workloads.freqs_table(64, start_pos + S + 1)
    latent = torch.randn(B, offset + T, Dqk, generator=g).bfloat16()
    q_att = torch.randn(B, S, Ha, Dqk, generator=g).bfloat16()
    sink = torch.randn(Ha, generator=g)
    print(f"[case] compressed chain start_pos={start_pos} offset={offset} T={T}", flush=True)
    kd = kcache.to(device)
    idx = ops.indexer(q_idx.to(device), kd[:, :T], w.to(device), tab.to(device), k_top, True, start_pos, ratio,
                      offset, 0, 64, False, T=T)
    assert idx.dtype == torch.int32
    out = ops.sparse_attn(q_att.to(device), latent.to(device), sink.to(device), idx, Dqk ** -0.5, dv=Dv)
    torch.cuda.synchronize()
    want_idx = oracle.indexer(bits(q_idx), bits(kcache[:, :T].contiguous()), w.numpy(), tab.numpy(), k_top, True,
                              start_pos, ratio, offset, 0, 64, False)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), want_idx)
    valid = want_idx >= 0
    assert (~valid).any() or start_pos > 0  # the prefill case has masked slots for its early queries
    assert (want_idx[valid] >= offset).all() and (want_idx[valid] < offset + T).all()
    want = oracle.sparse_attn(bits(q_att), bits(latent), sink.numpy(), want_idx.astype(np.int32), Dqk ** -0.5, dv=Dv)
    got = out.float().cpu().numpy()
    assert got.shape == (B, S, Ha, Dv)
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
