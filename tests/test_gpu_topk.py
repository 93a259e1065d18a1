"""GPU parity: exact top-k kernel vs the stable-sort oracle (bit-exact indices).

Covers the reference's TopK probe cases (optimized/indexer_project/design.md:163-167: heavy ties, rows
with fewer valid entries than k, garbage padding beyond the valid prefix, row counts that are not a
multiple of any block size) plus -inf blocks, signed zeros and every key-width variant."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import ops

pytestmark = pytest.mark.gpu


def _check(scores, k, causal=False, start_pos=0, ratio=1, offset=0, T=None, out_dtype=torch.int64):
    B, S, ld = scores.shape
    T = ld if T is None else T
    print(f"[case] topk B={B} S={S} T={T} ld={ld} k={k} causal={causal} start={start_pos} ratio={ratio}", flush=True)
    got = ops.topk_mask(scores, causal, ratio, T, offset, k=k, start_pos=start_pos, out_dtype=out_dtype)
    torch.cuda.synchronize()
    sc = scores[..., :T].cpu().numpy().copy()
    if causal:
        lim = (start_pos + np.arange(S) + 1) // ratio
        cols = np.arange(T)
        sc = np.where(cols[None, None, :] >= lim[None, :, None], np.float32(-np.inf), sc)
    kk = min(k, T)
    want = oracle.postprocess(oracle.topk_stable(sc, kk), causal, start_pos, ratio, offset)
    np.testing.assert_array_equal(got.cpu().numpy().astype(np.int64), want)


@pytest.mark.parametrize("T,k", [(1, 1), (7, 3), (100, 100), (1024, 128), (1500, 512), (4096, 512), (4096, 4096),
                                 (8192, 2048), (20000, 1000), (32768, 2048), (40000, 129), (65536, 3000)])
def test_topk_random_fp32(device, T, k):
    g = torch.Generator(device=device).manual_seed(T + k)
    s = torch.randn(2, 5, T, device=device, generator=g)
    _check(s, k)


@pytest.mark.parametrize("T,k", [(4096, 512), (32768, 2048), (650, 128)])
def test_topk_heavy_ties_bf16_values(device, T, k):
    # bf16-valued scores: ~1-2k distinct values per row, many exact ties at the threshold
    g = torch.Generator(device=device).manual_seed(T)
    s = torch.randn(3, 4, T, device=device, generator=g).bfloat16().float()
    _check(s, k)
    # coarse quantisation: every row is mostly ties
    q = torch.round(torch.randn(2, 3, T, device=device, generator=g) * 2) / 2
    _check(q.contiguous(), k)


def test_topk_all_equal_neg_inf_and_zeros(device):
    T = 3000
    s = torch.full((1, 4, T), -float("inf"), device=device)
    s[0, 1] = 1.0
    s[0, 2, :1000] = 0.0
    s[0, 2, 1000:2000] = -0.0
    s[0, 3, ::2] = 2.0
    _check(s, 1024)
    _check(s, 2999)


@pytest.mark.parametrize("T,k", [(1000, 128), (64, 64), (65, 1), (513, 97)])
def test_topk_short_rows_ties_and_neg_inf(device, T, k):
    # the one-wave-per-row path (T <= 1024, k <= 128): all -inf rows, +0/-0 ties, a single finite value,
    # alternating duplicates, rows of few distinct values, and more rows than one workgroup holds
    s = torch.full((3, 7, T), -float("inf"), device=device)
    s[0, 1] = 1.0
    s[0, 2, : T // 3] = 0.0
    s[0, 2, T // 3: 2 * T // 3] = -0.0
    s[0, 3, ::2] = 2.0
    s[1, 4, T - 1] = 5.0
    g = torch.Generator(device=device).manual_seed(T)
    s[2] = torch.round(torch.randn(7, T, device=device, generator=g))
    _check(s.contiguous(), k)
    _check(s.contiguous(), k, causal=True, start_pos=3, ratio=2, offset=9)


def test_topk_causal_limits_and_garbage_padding(device):
    # causal rows with limits below k (outputs -1), garbage beyond the limit must be ignored
    S, T = 40, 650
    g = torch.Generator(device=device).manual_seed(3)
    s = torch.randn(2, S, T, device=device, generator=g) * 100  # garbage everywhere
    _check(s, 128, causal=True, start_pos=0, ratio=4, offset=17)
    _check(s, 128, causal=True, start_pos=300, ratio=1, offset=0)
    _check(s, 600, causal=True, start_pos=600, ratio=1, offset=5, out_dtype=torch.int32)


@pytest.mark.parametrize("start_pos", [0, 1500])
def test_topk_wave_bf16_causal_prefixes(device, start_pos):
    # the drop-in geometry (650 columns, ratio 4, k = 128) with bf16-valued scores: rows whose valid prefix is at
    # most k (every valid column taken), prefixes ending inside a column group, and rows with exact ties at the
    # threshold; then the same rows with one non-bf16 value per row, which needs all four radix passes
    S, T = 700, 650
    g = torch.Generator(device=device).manual_seed(start_pos + 11)
    s = (torch.round(torch.randn(2, S, T, device=device, generator=g) * 8) / 8).bfloat16().float()
    _check(s.contiguous(), 128, causal=True, start_pos=start_pos, ratio=4, offset=3)
    s[:, :, 0] += 1.0 / 3.0  # not a bf16 value for any multiple of 1/8
    _check(s.contiguous(), 128, causal=True, start_pos=start_pos, ratio=4, offset=3)


def test_topk_leading_dimension_and_odd_rows(device):
    g = torch.Generator(device=device).manual_seed(4)
    base = torch.randn(3, 37, 1000, device=device, generator=g)
    _check(base, 77, T=900)  # ld = 1000 > T = 900


def test_topk_errors(device):
    s = torch.zeros(1, 2, 10, device=device)
    with pytest.raises(RuntimeError):
        ops.topk_mask(s.double(), False, 1, 10, 0, k=3)
    with pytest.raises(RuntimeError):
        ops.topk_mask(torch.zeros(1, 2, 10000, device=device), False, 1, 10000, 0, k=5000)
