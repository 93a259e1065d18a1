"""Pin the CPU oracle against mathematics that does not share its code.

CPU only (no GPU marker): exact rational arithmetic, brute force on tiny inputs,
closed forms and invariants.  A plausible oracle mistake (a dropped term, a wrong
rounding, a transposed operand, a wrong tie order) fails one of these.
"""
import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_ref
from tests import exact


# ------------------------------------------------------------------ exact dot
def _rand_bf16(rng, n, emin=-20, emax=6, zero_frac=0.0):
    m = rng.integers(0, 128, n)
    e = rng.integers(emin, emax, n)
    s = rng.integers(0, 2, n)
    bits = ((s << 15) | (((e + 127) & 0xFF) << 7) | m).astype(np.uint16)
    if zero_frac:
        bits[rng.random(n) < zero_frac] = 0
    return bits


def _exact_dot_bits(a, b):
    v = sum((exact.bf16_value(int(x)) * exact.bf16_value(int(y)) for x, y in zip(a, b)), Fraction(0))
    return exact.to_bf16_bits(exact.round_bf16(v))


def test_dot_exact_random_vs_fraction():
    rng = np.random.default_rng(1)
    for trial in range(300):
        n = int(rng.integers(1, 160))
        a = _rand_bf16(rng, n, zero_frac=0.1)
        b = _rand_bf16(rng, n, zero_frac=0.1)
        assert oracle.dot_exact(a, b) == _exact_dot_bits(a, b), trial


def test_dot_exact_wide_exponent_spread_big_path():
    # exponents spread over >96 bits force the multi-limb accumulator
    rng = np.random.default_rng(2)
    for trial in range(100):
        n = int(rng.integers(2, 40))
        a = _rand_bf16(rng, n, emin=-120, emax=100)
        b = _rand_bf16(rng, n, emin=-120, emax=20)
        assert oracle.dot_exact(a, b) == _exact_dot_bits(a, b), trial


def test_dot_exact_cancellation_and_ties():
    f = oracle.f32_to_bf16
    one = f(np.float32([1.0]))[0]
    cases = []
    # 1 + 2^-8: exactly halfway between 1 and 1+2^-7 -> ties to even -> 1
    cases.append(([1.0, 2.0 ** -8], [1.0, 1.0], 1.0))
    # 1 + 2^-7 + 2^-8: halfway between 1+2^-7 (odd) and 1+2^-6 (even) -> up
    cases.append(([1.0, 2.0 ** -7, 2.0 ** -8], [1.0, 1.0, 1.0], 1.0 + 2.0 ** -6))
    # 1 + 2^-8 + 2^-40: just above the midpoint -> up
    cases.append(([1.0, 2.0 ** -8, 2.0 ** -20], [1.0, 1.0, 2.0 ** -20], 1.0 + 2.0 ** -7))
    # catastrophic cancellation: 2^20 - 2^20 + 3*2^-30
    cases.append(([2.0 ** 20, -(2.0 ** 20), 3.0 * 2 ** -30], [1.0, 1.0, 1.0], 3.0 * 2 ** -30))
    # exact zero -> +0
    cases.append(([2.0, -2.0], [3.0, 3.0], 0.0))
    for av, bv, want in cases:
        a = f(np.float32(av))
        b = f(np.float32(bv))
        got = oracle.bf16_to_f32(np.uint16(oracle.dot_exact(a, b)))
        assert float(got) == want, (av, bv, float(got), want)
    assert one == 0x3F80
    # +0 bits for exact cancellation
    assert oracle.dot_exact(f(np.float32([2.0, -2.0])), f(np.float32([3.0, 3.0]))) == 0


def test_dot_exact_subnormal_results():
    # products near the bf16 subnormal range: 2^-70 * 2^-62 = 2^-132
    f = oracle.f32_to_bf16
    a = f(np.float32([2.0 ** -70, 2.0 ** -70]))
    b = f(np.float32([2.0 ** -62, 2.0 ** -63]))
    want = _exact_dot_bits(a, b)
    assert oracle.dot_exact(a, b) == want
    assert want & 0x7F80 == 0  # really subnormal


def test_dot_matrix_matches_single():
    rng = np.random.default_rng(3)
    A = oracle.f32_to_bf16(rng.standard_normal((5, 128)).astype(np.float32))
    B = oracle.f32_to_bf16(rng.standard_normal((7, 128)).astype(np.float32))
    M = oracle.dot_matrix(A, B, threads=2)
    for i in range(5):
        for j in range(7):
            assert M[i, j] == _exact_dot_bits(A[i], B[j])


# ------------------------------------------------------------------ scores
def _scores_fraction(q, k, w, causal, start_pos, ratio):
    """Canonical order recomputed with Fractions and explicit roundings."""
    B, S, H, D = q.shape
    T = k.shape[1]
    out = np.empty((B, S, T), dtype=np.float32)
    bfw = w.dtype == np.uint16
    for b in range(B):
        for s in range(S):
            lim = (start_pos + s + 1) // ratio
            for t in range(T):
                if causal and t >= lim:
                    out[b, s, t] = -np.inf
                    continue
                G = [Fraction(0)] * 4
                for h in range(H):
                    d = exact.round_bf16(sum((exact.bf16_value(int(x)) * exact.bf16_value(int(y))
                                              for x, y in zip(q[b, s, h], k[b, t])), Fraction(0)))
                    r = d if d > 0 else Fraction(0)
                    g = (h // 4) % 4
                    if bfw:
                        wh = exact.bf16_value(int(w[b, s, h]))
                        G[g] = exact.round_f32(G[g] + exact.round_bf16(r * wh))
                    else:
                        wh = exact.f32_value(float(w[b, s, h]))
                        G[g] = exact.round_f32(r * wh + G[g])  # one rounding: fma
                sc = exact.round_f32(exact.round_f32(G[0] + G[1]) + exact.round_f32(G[2] + G[3]))
                if bfw:
                    sc = exact.round_bf16(sc)
                out[b, s, t] = exact.to_f32(sc)
    return out


@pytest.mark.parametrize("w_bf16", [False, True])
def test_indexer_scores_canonical_order(w_bf16):
    rng = np.random.default_rng(4)
    B, S, H, D, T = 1, 3, 16, 8, 6
    q = oracle.f32_to_bf16(rng.standard_normal((B, S, H, D)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((B, T, D)).astype(np.float32))
    wf = (rng.standard_normal((B, S, H)) / 8).astype(np.float32)
    w = oracle.f32_to_bf16(wf) if w_bf16 else wf
    got = oracle.indexer_scores(q, k, w, causal=True, start_pos=2, ratio=1)
    want = _scores_fraction(q, k, w, True, 2, 1)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_indexer_scores_single_head_closed_form():
    rng = np.random.default_rng(5)
    q = oracle.f32_to_bf16(rng.standard_normal((1, 4, 1, 32)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((1, 9, 32)).astype(np.float32))
    w = (rng.standard_normal((1, 4, 1))).astype(np.float32)
    got = oracle.indexer_scores(q, k, w, causal=False, start_pos=0)
    d = oracle.bf16_to_f32(oracle.dot_matrix(q[0, :, 0], k[0]))
    want = np.maximum(d, np.float32(0)) * w[0, :, 0][:, None]  # one rounding = fma(r, w, +0)
    np.testing.assert_array_equal(got[0], want.astype(np.float32))


def test_indexer_scores_mask_closed_form():
    rng = np.random.default_rng(6)
    B, S, H, D, T = 2, 5, 16, 16, 12
    q = oracle.f32_to_bf16(rng.standard_normal((B, S, H, D)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((B, T, D)).astype(np.float32))
    w = rng.standard_normal((B, S, H)).astype(np.float32)
    for start_pos, ratio in [(0, 1), (7, 1), (0, 4), (40, 4)]:
        sc = oracle.indexer_scores(q, k, w, True, start_pos, ratio)
        for s in range(S):
            lim = (start_pos + s + 1) // ratio
            assert np.all(np.isneginf(sc[:, s, lim:]))
            assert np.all(np.isfinite(sc[:, s, :min(lim, T)]))
    # negative dots vanish under relu: negate k -> only the other half of dots count
    sc_pos = oracle.indexer_scores(q, k, np.abs(w), False, 0)
    assert np.all(sc_pos >= 0)


# ------------------------------------------------------------------ RoPE
def test_rope_position_zero_identity_and_unit_vectors():
    tab = oracle.freqs_table(64, 16)
    rng = np.random.default_rng(7)
    x = oracle.f32_to_bf16(rng.standard_normal((1, 1, 3, 128)).astype(np.float32))
    y = oracle.rope_bf16(x, tab, 0, 64, pos0=0)
    np.testing.assert_array_equal(x, y)
    # unit vector (1, 0) at each position p -> (cos, sin) rounded to bf16
    e = np.zeros((1, 16, 1, 128), dtype=np.float32)
    e[..., 0:64:2] = 1.0
    out = oracle.bf16_to_f32(oracle.rope_bf16(oracle.f32_to_bf16(e), tab, 0, 64, pos0=0))
    np.testing.assert_array_equal(out[0, :, 0, 0:64:2], oracle.bf16_to_f32(oracle.f32_to_bf16(tab[:, :, 0])))
    np.testing.assert_array_equal(out[0, :, 0, 1:64:2], oracle.bf16_to_f32(oracle.f32_to_bf16(tab[:, :, 1])))
    # dims outside the rotated segment are untouched
    np.testing.assert_array_equal(out[..., 64:], 0)


def test_rope_matches_complex128_and_inverse():
    tab = oracle.freqs_table(64, 4096)
    rng = np.random.default_rng(8)
    x = oracle.f32_to_bf16(rng.standard_normal((1, 64, 4, 128)).astype(np.float32))
    y = oracle.rope_bf16(x, tab, 64, 64, pos0=1000)  # rotate the LAST 64 dims, positions 1000..
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    z = (xf[..., 64::2] + 1j * xf[..., 65::2]) * (tab[1000:1064, None, :, 0] + 1j * tab[1000:1064, None, :, 1])
    yf = oracle.bf16_to_f32(y).astype(np.float64)
    # within one bf16 ulp of the complex128 product
    tol = np.abs(z) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(yf[..., 64::2] - z.real) <= tol)
    assert np.all(np.abs(yf[..., 65::2] - z.imag) <= tol)
    # inverse rotation (conjugate table) composes to ~identity
    inv = tab.copy()
    inv[..., 1] = -inv[..., 1]
    back = oracle.bf16_to_f32(oracle.rope_bf16(y, inv, 64, 64, pos0=1000)).astype(np.float64)
    assert np.max(np.abs(back - xf)) < 0.05


# ------------------------------------------------------------------ TopK
def _topk_bruteforce(v, k):
    """Lexicographically greatest k-permutation under key (value, -index) per slot."""
    best = None
    for perm in itertools.permutations(range(len(v)), k):
        key = [(v[i], -i) for i in perm]
        if best is None or key > best[0]:
            best = (key, perm)
    return list(best[1])


def test_topk_bruteforce_with_ties_and_neg_inf():
    rng = np.random.default_rng(9)
    vals = np.array([-np.inf, -1.0, 0.0, 0.5, 0.5, 2.0], dtype=np.float32)
    for trial in range(200):
        n = int(rng.integers(1, 7))
        k = int(rng.integers(1, n + 1))
        v = rng.choice(vals, n)
        got = oracle.topk_stable(v[None, :], k)[0].tolist()
        assert got == _topk_bruteforce(v.tolist(), k), (v, k, got)


def test_topk_all_equal_and_all_masked():
    v = np.full((2, 10), -np.inf, dtype=np.float32)
    v[1] = 3.0
    np.testing.assert_array_equal(oracle.topk_stable(v, 4), [[0, 1, 2, 3], [0, 1, 2, 3]])


def test_postprocess_closed_form():
    idx = np.array([[[0, 1, 2]], [[5, 9, 3]]], dtype=np.int64).reshape(1, 2, 3)
    # S=2, start_pos=0, ratio=4: limits (0+1)//4=0 and (0+2)//4=0 -> everything -1
    np.testing.assert_array_equal(oracle.postprocess(idx, True, 0, 4, 100), -np.ones_like(idx))
    # start_pos=10, ratio=1: limits 11, 12 -> 9,5,3 kept (+100), none invalid
    np.testing.assert_array_equal(oracle.postprocess(idx, True, 10, 1, 100), idx + 100)
    # start_pos=3, ratio=1: limits 4 and 5 -> row0 [0,1,2]+100; row1 5->-1, 9->-1, 3->103
    got = oracle.postprocess(idx, True, 3, 1, 100)
    np.testing.assert_array_equal(got, [[[100, 101, 102], [-1, -1, 103]]])
    np.testing.assert_array_equal(oracle.postprocess(idx, False, 3, 1, 7), idx + 7)


def test_indexer_end_to_end_vs_torch_cpu_sets():
    """The canonical oracle and the plain torch-CPU op sequence pick (almost) the same sets."""
    g = torch.Generator().manual_seed(10)
    B, S, H, D, T, kt = 1, 8, 16, 128, 256, 32
    q = torch.randn(B, S, H, D, generator=g).bfloat16()
    k = torch.randn(B, T, D, generator=g).bfloat16()
    w = torch.randn(B, S, H, generator=g) / 8
    tab = oracle.freqs_table(64, 512)
    cis = torch.view_as_complex(torch.from_numpy(tab).contiguous())
    sp = T - S
    a = oracle.indexer(q.view(torch.int16).numpy().view(np.uint16), k.view(torch.int16).numpy().view(np.uint16),
                       w.numpy(), tab, kt, True, sp, 1, 0)
    b = torch_ref.indexer(q, k, w, cis, kt, True, sp, 1, 0).numpy()
    overlap = np.mean([len(set(a[0, s]) & set(b[0, s])) / kt for s in range(S)])
    assert overlap > 0.97


# ------------------------------------------------------------------ Sinkhorn
def test_sinkhorn_constant_input_closed_form():
    x = np.zeros((3, 4, 4), dtype=np.float32)
    y = oracle.sinkhorn(x, repeat=10, eps=1e-6)
    np.testing.assert_allclose(y, 0.25, atol=1e-5)


def test_sinkhorn_invariants_and_equivariance():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 4, 4)).astype(np.float32)
    y = oracle.sinkhorn(x, 10, 1e-6)
    assert np.all(y > 0)
    np.testing.assert_allclose(y.sum(axis=-2), 1.0, atol=1e-5)
    np.testing.assert_allclose(y.sum(axis=-1), 1.0, atol=2e-3)
    pr, pc = rng.permutation(4), rng.permutation(4)
    yp = oracle.sinkhorn(x[:, pr][:, :, pc], 10, 1e-6)
    np.testing.assert_allclose(yp, y[:, pr][:, :, pc], atol=1e-12)
    # fp32 torch restatement agrees
    yt = torch_ref.sinkhorn(torch.from_numpy(x), 10, 1e-6).numpy()
    np.testing.assert_allclose(yt, y, atol=1e-5, rtol=1e-5)


def test_sinkhorn_rational_closed_forms_pin_eps_and_iteration_count():
    # x = log(m): the softmax of a row is m / rowsum exactly, so with a rational eps every step is rational.
    # repeat = 1 is softmax (+ eps) then one column normalisation; the values below were derived by hand
    # (row 0 of m sums to 8, so its softmax is [1, 2, 1, 4] / 8; column 0 then sums to 37/40; ...).
    from fractions import Fraction as Fr
    m = np.array([[1, 2, 1, 4], [3, 1, 1, 1], [2, 2, 5, 1], [1, 6, 1, 2]], dtype=np.float64)
    x = np.log(m)[None]
    one = {Fr(0): [["5/37", "15/73", "15/107", "15/29"], ["20/37", "10/73", "20/107", "5/29"],
                   ["8/37", "12/73", "60/107", "3/29"], ["4/37", "36/73", "12/107", "6/29"]],
           Fr(1, 4): [["5/29", "15/74", "45/257", "45/133"], ["10/29", "25/148", "50/257", "25/133"],
                      ["6/29", "27/148", "90/257", "3/19"], ["14/87", "51/148", "42/257", "27/133"]]}
    for eps, lit in one.items():
        want1 = [[Fr(v) for v in row] for row in lit]
        np.testing.assert_allclose(oracle.sinkhorn(x, 1, float(eps))[0], np.array(want1, dtype=np.float64),
                                   rtol=1e-13, atol=0)
        # one more iteration is one row normalisation then one column normalisation of that matrix (each
        # dividing by the sum + eps), done here in exact rationals
        rs = [sum(r) + eps for r in want1]
        v = [[want1[i][j] / rs[i] for j in range(4)] for i in range(4)]
        cs = [sum(v[i][j] for i in range(4)) + eps for j in range(4)]
        want2 = [[v[i][j] / cs[j] for j in range(4)] for i in range(4)]
        got2 = oracle.sinkhorn(x, 2, float(eps))[0]
        np.testing.assert_allclose(got2, np.array([[float(a) for a in r] for r in want2]), rtol=1e-13, atol=0)
        # and repeat = 2 is not repeat = 1 or 3 (the count is what the check sees)
        assert np.abs(got2 - oracle.sinkhorn(x, 1, float(eps))[0]).max() > 1e-3
        assert np.abs(got2 - oracle.sinkhorn(x, 3, float(eps))[0]).max() > 1e-4


# ------------------------------------------------------------------ sparse attention
def _bf(a):
    return oracle.f32_to_bf16(np.asarray(a, dtype=np.float32))


def test_sparse_attn_closed_forms():
    rng = np.random.default_rng(12)
    B, M, H, D, N, K = 1, 3, 4, 16, 10, 5
    q = _bf(rng.standard_normal((B, M, H, D)))
    kv = _bf(rng.standard_normal((B, N, D)))
    sink = np.zeros(H, dtype=np.float32)
    # all invalid -> 0
    idx = -np.ones((B, M, K), dtype=np.int32)
    np.testing.assert_array_equal(oracle.sparse_attn(q, kv, sink, idx, 0.25), 0.0)
    # equal scores (q = 0) -> k/(k + e^(sink - 0)) * mean(V)
    q0 = np.zeros_like(q)
    idx = rng.integers(0, N, (B, M, K)).astype(np.int32)
    out = oracle.sparse_attn(q0, kv, sink, idx, 0.25)
    kvf = oracle.bf16_to_f32(kv).astype(np.float64)
    for m in range(M):
        mean = kvf[0, idx[0, m]].mean(axis=0)
        np.testing.assert_allclose(out[0, m], np.broadcast_to(K / (K + 1.0) * mean, (H, D)), rtol=1e-12, atol=1e-12)
    # single valid index with sink -> -inf: exactly that row
    idx = -np.ones((B, M, K), dtype=np.int32)
    idx[0, :, 2] = [4, 7, 1]
    out = oracle.sparse_attn(q, kv, np.full(H, -np.inf, dtype=np.float32), idx, 0.25)
    for m, r in enumerate([4, 7, 1]):
        np.testing.assert_allclose(out[0, m], np.broadcast_to(kvf[0, r], (H, D)), rtol=0, atol=0)
    # duplicates count with multiplicity: [r, r, s] == weights 2:1 at equal scores
    idx = np.array([[[3, 3, 6]]], dtype=np.int32)
    out = oracle.sparse_attn(np.zeros((1, 1, H, D), np.uint16), kv, sink, idx, 1.0)
    want = (2 * kvf[0, 3] + kvf[0, 6]) / 4.0
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(want, (H, D)), rtol=1e-12)


def test_sparse_attn_two_key_closed_form_pins_scale():
    # one head, two valid keys: s_i = scale * q.k_i, and with a sink the output is
    #   (e^s1 v1 + e^s2 v2) / (e^s1 + e^s2 + e^sink),  v_i = k_i (K = V = kv)
    # q = 2 e_0, k1 = e_0 + 3 e_1, k2 = -e_1 + 5 e_2: s1 = 2 scale, s2 = 0 (every value exact in bf16)
    D = 16
    q = np.zeros((1, 1, 1, D), np.float32)
    q[0, 0, 0, 0] = 2.0
    kv = np.zeros((1, 2, D), np.float32)
    kv[0, 0, 0], kv[0, 0, 1] = 1.0, 3.0
    kv[0, 1, 1], kv[0, 1, 2] = -1.0, 5.0
    idx = np.array([[[0, 1]]], dtype=np.int32)
    v1, v2 = kv[0, 0].astype(np.float64), kv[0, 1].astype(np.float64)
    for scale in (0.3, 128 ** -0.5, 576 ** -0.5, 1.7):
        for sink in (-np.inf, 0.0, 0.7):
            e1, e2, es = np.exp(2 * scale), 1.0, np.exp(np.float64(np.float32(sink)))  # the sink is fp32
            want = (e1 * v1 + e2 * v2) / (e1 + e2 + es)
            got = oracle.sparse_attn(_bf(q), _bf(kv), np.array([sink], np.float32), idx, scale)[0, 0, 0]
            np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-15)
    # the output moves with the scale: a scale off by any factor is seen
    a = oracle.sparse_attn(_bf(q), _bf(kv), np.zeros(1, np.float32), idx, 0.3)
    b = oracle.sparse_attn(_bf(q), _bf(kv), np.zeros(1, np.float32), idx, 0.6)
    assert np.abs(a - b).max() > 0.05


def test_sparse_attn_matches_torch_cpu():
    g = torch.Generator().manual_seed(13)
    B, M, H, D, N, K = 2, 4, 8, 64, 40, 12
    q = torch.randn(B, M, H, D, generator=g).bfloat16()
    kv = torch.randn(B, N, D, generator=g).bfloat16()
    idx = torch.randint(-3, N, (B, M, K), generator=g, dtype=torch.int32)
    sink = torch.randn(H, generator=g)
    a = oracle.sparse_attn(q.view(torch.int16).numpy().view(np.uint16), kv.view(torch.int16).numpy().view(np.uint16),
                           sink.numpy(), idx.numpy(), D ** -0.5, dv=48)
    b = torch_ref.sparse_attn(q, kv, sink, idx, D ** -0.5, dv=48).float().numpy()
    np.testing.assert_allclose(b, a, atol=1e-2, rtol=1e-2)


# ------------------------------------------------------------------ agreement with the reference's arithmetic
def test_agreement_with_reference_arithmetic_fp32_weights():
    """Index lists of the canonical contract and of the reference's torch op sequence differ only where two
    keys' scores lie within one rounding per dot of each other (tests/agreement.py states the tolerance)."""
    from tests import agreement
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 48, 64, 128, generator=g).bfloat16()
    k = torch.randn(1, 900, 128, generator=g).bfloat16()
    w = torch.randn(1, 48, 64, generator=g) / 8
    r = agreement.compare(q, k, w, oracle.freqs_table(64, 1024), 128, True, 900 - 48)
    assert r["positions_within_rounding"] == r["mismatched_positions"]
    assert r["set_differences_within_rounding"] == r["set_differences"]
    assert r["set_overlap"] > 0.99


def test_agreement_with_reference_arithmetic_bf16_weights():
    """With bf16 weights (the drop-in's) the reference's scores are bf16; every position where the lists
    differ holds two keys whose reference scores are exactly equal (CPU torch.topk orders ties arbitrarily)."""
    from tests import agreement
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 64, 16, 64, generator=g).bfloat16()
    k = torch.randn(1, 650, 64, generator=g).bfloat16()
    w = (torch.randn(1, 64, 16, generator=g) / 8).bfloat16()
    r = agreement.compare(q, k, w, oracle.freqs_table(32, 1024), 128, True, 650 - 64, 1, 32, 32, False)
    assert r["mismatched_positions"] > 0  # ties do occur at this shape
    assert r["positions_tied_in_reference_score"] == r["mismatched_positions"]
    assert r["set_differences_within_rounding"] == r["set_differences"]


def test_freqs_table_against_the_mathematics():
    """oracle.freqs_table (baseline/indexer.py:226-235) against fp64 cos/sin: the fp32 inverse frequencies
    are within 2^-22 of theta^(-2j/d), every angle is the fp32 rounding of position x inverse frequency,
    the (cos, sin) pairs are within 2^-23 of the fp64 values of those angles, and within the angle's own
    rounding of the textbook cos/sin(p theta^(-2j/d)); position 0 is (1, 0) exactly."""
    d, n = 64, 4096
    tab = oracle.freqs_table(d, n).astype(np.float64)
    assert tab.shape == (n, d // 2, 2)
    j = np.arange(d // 2)
    inv_exact = 10000.0 ** (-2.0 * j / d)
    inv32 = (1.0 / (10000.0 ** (torch.arange(0, d, 2).float() / d))).numpy()  # the reference's fp32 formula
    assert np.all(np.abs(inv32.astype(np.float64) / inv_exact - 1) < 2.0 ** -22)
    p = np.arange(n, dtype=np.float64)[:, None]
    ang32 = (p.astype(np.float32) * inv32[None, :]).astype(np.float64)  # fp32 product, as torch.outer
    np.testing.assert_allclose(tab[..., 0], np.cos(ang32), rtol=0, atol=2.0 ** -23)
    np.testing.assert_allclose(tab[..., 1], np.sin(ang32), rtol=0, atol=2.0 ** -23)
    ang = p * inv_exact[None, :]
    err = np.abs(ang32 - ang) + 2.0 ** -23
    assert np.all(np.abs(tab[..., 0] - np.cos(ang)) <= err + 2.0 ** -23)
    assert np.all(np.abs(tab[..., 1] - np.sin(ang)) <= err + 2.0 ** -23)
    np.testing.assert_array_equal(tab[0, :, 0], 1.0)
    np.testing.assert_array_equal(tab[0, :, 1], 0.0)
    # a table with a dropped factor of 2 in the exponent or swapped (cos, sin) fails the checks above
    bad = np.stack([np.cos(p * 10000.0 ** (-1.0 * j / d)), np.sin(p * 10000.0 ** (-1.0 * j / d))], -1)
    assert np.max(np.abs(bad - tab)) > 0.1
    assert np.max(np.abs(tab[..., ::-1] - tab)) > 0.1


# ------------------------------------------------------------------ mHC hyper-connections
def test_mhc_oracle_closed_forms():
    rng = np.random.default_rng(5)
    N, C = 6, 16
    x = oracle.f32_to_bf16(rng.standard_normal((N, 4, C)).astype(np.float32))
    f = oracle.f32_to_bf16(rng.standard_normal((N, C)).astype(np.float32))
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    ff = oracle.bf16_to_f32(f).astype(np.float64)
    # constant residual logits: the doubly stochastic matrix is 1/4 everywhere (up to eps) -> stream mean
    out = oracle.mhc_post(x, f, np.zeros((N, 4, 4), np.float32), np.zeros((N, 4), np.float32), 20, 1e-6)
    np.testing.assert_allclose(out, np.broadcast_to(xf.mean(1, keepdims=True) + ff[:, None, :], out.shape),
                               rtol=1e-5, atol=1e-5)
    # zero pre logits: sigmoid 1/2 on every stream
    np.testing.assert_allclose(oracle.mhc_pre(x, np.zeros((N, 4), np.float32)), 0.5 * xf.sum(1), rtol=1e-12)
    # very negative post logits switch the layer output off; a permutation of the residual logits' rows
    # permutes the output streams (the Sinkhorn is equivariant)
    res = rng.standard_normal((N, 4, 4)).astype(np.float32)
    off = np.full((N, 4), -200.0, np.float32)
    a = oracle.mhc_post(x, f, res, off, 20, 1e-6)
    perm = [2, 0, 3, 1]
    b = oracle.mhc_post(x, f, res[:, perm, :], off, 20, 1e-6)
    np.testing.assert_allclose(b, a[:, perm, :], rtol=1e-12, atol=1e-12)
    # the mixing matrix is the Sinkhorn oracle's, applied as a plain matrix product
    S = oracle.sinkhorn(res, 20, 1e-6)
    np.testing.assert_allclose(a, np.einsum("nij,njc->nic", S, xf), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ FP8 rows
def _torch_e4m3(y):
    return torch.from_numpy(np.ascontiguousarray(y, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _e4m3_values():
    """All finite e4m3fn values (nonnegative codes 0x00..0x7E), by their definition."""
    out = []
    for c in range(0x7F):
        e, m = c >> 3, c & 7
        out.append(Fraction(m, 512) if e == 0 else Fraction(8 + m, 8) * Fraction(2) ** (e - 7))
    return out


def test_e4m3_encode_against_torch_and_bruteforce():
    # every bf16 value in range
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(b)
    y = f[np.isfinite(f) & (np.abs(f) <= 448)]
    np.testing.assert_array_equal(oracle.e4m3_encode(y), _torch_e4m3(y))
    # every midpoint between neighbouring codes (a tie: the even code wins), and its fp32 neighbours
    vals = _e4m3_values()
    mids = np.array([float((a + c) / 2) for a, c in zip(vals[:-1], vals[1:])], np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    near = np.concatenate([near, -near])
    np.testing.assert_array_equal(oracle.e4m3_encode(near), _torch_e4m3(near))
    # brute force: nearest value, ties to the even code (pure Python over a sample)
    rng = np.random.default_rng(7)
    sample = np.concatenate([mids[::3], (rng.random(300) * 448).astype(np.float32),
                             (2.0 ** rng.uniform(-12, -5, 200)).astype(np.float32)])
    for v in sample:
        x = Fraction(float(v))
        best = min(range(0x7F), key=lambda c: (abs(vals[c] - x), c & 1))
        assert int(oracle.e4m3_encode(np.float32(v))) == best, v
    assert int(oracle.e4m3_encode(np.float32(-0.0))) == 0x80
    assert int(oracle.e4m3_encode(np.float32(448.0))) == 0x7E


def test_e4m3_decode_all_codes():
    c = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(c.copy()).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(oracle.e4m3_decode(c), want)  # NaN codes compare equal as NaN
    vals = _e4m3_values()
    assert [Fraction(float(v)) for v in oracle.e4m3_decode(c[:0x7F])] == vals


@pytest.mark.parametrize("block,ue8m0", [(128, True), (128, False), (32, True), (8, False)])
def test_fp8_quant_rows_closed_forms(block, ue8m0):
    rng = np.random.default_rng(block + ue8m0)
    rows, D = 64, 256
    x = rng.standard_normal((rows, D)) * 2.0 ** rng.integers(-20, 20, (rows, 1))
    x[3] = 0.0                                      # all-zero row: the 1e-4 floor
    x[4, :block] = 1.0 + 1.0 / 16                   # e4m3 ties once scaled by a power of two
    xb = oracle.f32_to_bf16(x.astype(np.float32))
    codes, s = oracle.fp8_quant_rows(xb, block, ue8m0)
    assert codes.shape == (rows, D) and s.shape == (rows, D // block) and s.dtype == np.float32
    xf = oracle.bf16_to_f32(xb).reshape(rows, D // block, block)
    amax = np.maximum(np.abs(xf).max(-1), np.float32(1e-4))
    if ue8m0:
        m, _ = np.frexp(s)
        assert (m == 0.5).all()                     # powers of two
        r = amax / s
        assert (r > 224 * (1 - 2.0 ** -20)).all() and (r <= 448 * (1 + 2.0 ** -20)).all()
    else:
        np.testing.assert_array_equal(s, (amax * np.float32(1 / np.float32(448))).astype(np.float32))
    # the codes are torch's cast of the clipped, scaled rows
    y = np.clip((xf / s[..., None]).astype(np.float32), -448, 448)
    np.testing.assert_array_equal(codes.reshape(rows, D // block, block), _torch_e4m3(y))
    # the element of largest magnitude lands in the top binade [256, 448]
    big = np.abs(oracle.e4m3_decode(codes).reshape(rows, D // block, block)).max(-1)
    live = np.abs(xf).max(-1) >= 1e-4
    assert (big[live] >= 224).all() and (big[live] <= 448).all()
    assert (codes[3] == 0).all()
    # dequantisation with power-of-two scales is exact: value(code) * s lands on the e4m3 grid times s
    if ue8m0:
        c2 = codes.reshape(-1, block)
        deq = oracle.bf16_to_f32(oracle.fp8_dequant_rows(c2, s.reshape(-1)))
        exact = [float(v) * float(sc) for v, sc in zip(oracle.e4m3_decode(c2).ravel(), np.repeat(s.ravel(), block))]
        np.testing.assert_array_equal(deq.ravel().astype(np.float64), np.array(exact))
