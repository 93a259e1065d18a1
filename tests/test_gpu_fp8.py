"""GPU parity: FP8 (e4m3fn) quantisation and the indexer on FP8 rows, bit-exact against the CPU oracle.

Quantisation codes and scales are compared bit for bit; the indexer's indices exactly, against the oracle
run on the dequantised rows, on shapes that take both score paths (bounded: 64 heads, D = 128, fp32
weights; exact: other shapes and bf16 weights), causal prefill and decode, compressed keys with an
offset, a batch-strided key cache, and at the config-2 shape against the bf16 indexer on the same
dequantised rows.  The last test pins the measured behaviour of the FP8 matrix instruction that keeps it
out of the exact score path."""
import numpy as np
import pytest
import torch

import oracle
from kernelswift_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu

bits = workloads.bf16_bits


def _rows(g, shape, spread=20):
    """bf16 rows N(0,1) with a per-row power-of-two scale in [2^-spread, 2^spread)."""
    x = torch.randn(*shape, generator=g)
    if spread == 0:
        return x.bfloat16()
    sc = 2.0 ** torch.randint(-spread, spread, (*shape[:-1], 1), generator=g).float()
    return (x * sc).bfloat16()


def _codes_np(c):
    return c.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("block,ue8m0", [(128, True), (128, False), (64, True), (32, False), (8, True)])
def test_fp8_quant_matches_oracle(device, block, ue8m0):
    g = torch.Generator().manual_seed(block * 2 + ue8m0)
    x = _rows(g, (517, 256))
    x[0] = 0                                  # the 1e-4 floor
    x[1, :] = 1.0625                          # e4m3 ties after scaling by a power of two
    x[2, ::2] = -448.0
    x[3, 5] = 3e38                            # a huge element next to tiny ones
    x[4] = 1e-38                              # bf16 subnormal-range rows
    print(f"[case] fp8 quant block={block} ue8m0={ue8m0}", flush=True)
    codes, s = ops.fp8_quant(x.to(device), block, ue8m0)
    torch.cuda.synchronize()
    want_c, want_s = oracle.fp8_quant_rows(bits(x), block, ue8m0)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    np.testing.assert_array_equal(_codes_np(codes), want_c)


def test_fp8_quant_torch_op(device):
    g = torch.Generator().manual_seed(5)
    x = _rows(g, (2, 7, 64, 128))
    print("[case] fp8 quant torch op", flush=True)
    codes, s = _lib.torch_ops().fp8_quant(x.to(device), 128, True)
    torch.cuda.synchronize()
    assert codes.dtype == torch.float8_e4m3fn and tuple(s.shape) == (2, 7, 64, 1)
    want_c, want_s = oracle.fp8_quant_rows(bits(x), 128, True)
    np.testing.assert_array_equal(_codes_np(codes), want_c)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)


def _quantised_inputs(g, device, B, S, H, D, Tk, spread=8):
    q = _rows(g, (B, S, H, D), spread)
    k = _rows(g, (B, Tk, D), spread)
    qc, qs = ops.fp8_quant(q.to(device), D, True)
    kc, ks_ = ops.fp8_quant(k.to(device), D, True)
    return qc, qs[..., 0].contiguous(), kc, ks_[..., 0].contiguous()


CASES = [
    # B, S, H, D, T, Tk, k_top, causal, start_pos, ratio, offset, w_bf16
    (2, 24, 64, 128, 300, 300, 64, True, 0, 1, 0, False),       # bounded path, prefill
    (1, 4, 64, 128, 2000, 2048, 512, True, 1996, 1, 0, False),  # bounded path, decode, spare cache rows
    (2, 16, 16, 64, 160, 200, 32, True, 600, 4, 128, False),    # exact path, compressed keys + offset
    (1, 33, 64, 128, 700, 700, 700, False, 0, 1, 5, True),      # exact path (bf16 weights), k_top = T
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_indexer_fp8_matches_oracle(device, case):
    B, S, H, D, T, Tk, k_top, causal, start_pos, ratio, offset, w_bf16 = case
    g = torch.Generator().manual_seed(sum(case[:7]))
    qc, qs, kc, ks_ = _quantised_inputs(g, device, B, S, H, D, Tk)
    w = torch.randn(B, S, H, generator=g) / 8
    w = w.bfloat16() if w_bf16 else w
    print(f"[case] indexer fp8 {case}", flush=True)
    out = ops.indexer_fp8(qc, qs, kc, ks_, w.to(device), k_top, causal, start_pos, ratio, offset,
                          out_dtype=torch.int64, T=T)
    torch.cuda.synchronize()
    w_np = bits(w) if w_bf16 else w.numpy()
    kc_np, ks_np = _codes_np(kc)[:, :T], ks_.cpu().numpy()[:, :T]
    want = oracle.indexer_fp8(_codes_np(qc), qs.cpu().numpy(), np.ascontiguousarray(kc_np),
                              np.ascontiguousarray(ks_np), w_np, k_top, causal, start_pos, ratio, offset)
    np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_indexer_fp8_batch_strided_cache_torch_op(device):
    # k codes and scales are views of a larger cache [4, 512, D] / [4, 512]: batch stride 512 rows
    g = torch.Generator().manual_seed(11)
    B, S, H, D, T = 2, 8, 64, 128, 384
    qc, qs, kc_all, ks_all = _quantised_inputs(g, device, 4, S, H, D, 512)
    qc, qs = qc[:B].contiguous(), qs[:B].contiguous()
    w = (torch.randn(B, S, H, generator=g) / 8).to(device)
    print("[case] indexer fp8 strided cache", flush=True)
    out = _lib.torch_ops().indexer_fp8(qc, qs, kc_all[:B], ks_all[:B], w, 128, True, T - S, 1, 0, False, T)
    torch.cuda.synchronize()
    assert out.dtype == torch.int32
    want = oracle.indexer_fp8(_codes_np(qc), qs.cpu().numpy(), np.ascontiguousarray(_codes_np(kc_all)[:B, :T]),
                              np.ascontiguousarray(ks_all.cpu().numpy()[:B, :T]), w.cpu().numpy(), 128, True, T - S)
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)


def _dbg_fp8(qc, qs, kc, ks_, w, k_top, causal, start_pos, path, T):
    B, S, H, D = qc.shape
    ws = torch.empty(ops.indexer_workspace_size(B, S, H, D, T), dtype=torch.uint8, device=qc.device)
    out = torch.empty(B, S, min(k_top, T), dtype=torch.int32, device=qc.device)
    rc = _lib.load().ks_dbg_indexer_fp8(qc.data_ptr(), qs.data_ptr(), kc.data_ptr(), ks_.data_ptr(), w.data_ptr(), 0,
                                        k_top, 1 if causal else 0, start_pos, 1, 0, out.data_ptr(), 0, B, S, H, D, T,
                                        kc.shape[1], ws.data_ptr(), ws.numel(),
                                        torch.cuda.current_stream().cuda_stream, None, path)
    _lib.check(rc, "ks_dbg_indexer_fp8")
    return out


def test_indexer_fp8_config2_equals_bf16_indexer(device):
    # config-2 shape (B=1, S=128, T=4096, 64 heads, D=128, k=512): the FP8 entry, its exact path, and the
    # bf16 indexer on the same dequantised rows (no RoPE) return identical indices
    g = torch.Generator().manual_seed(2)
    B, S, H, D, T, k_top = 1, 128, 64, 128, 4096, 512
    qc, qs, kc, ks_ = _quantised_inputs(g, device, B, S, H, D, T, spread=0)
    w = (torch.randn(B, S, H, generator=g) / 8).to(device)
    print("[case] indexer fp8 config-2 shape", flush=True)
    got = ops.indexer_fp8(qc, qs, kc, ks_, w, k_top, True, 0)
    exact = _dbg_fp8(qc, qs, kc, ks_, w, k_top, True, 0, 1, T)
    qd = torch.from_numpy(oracle.fp8_dequant_rows(_codes_np(qc), qs.cpu().numpy()).view(np.int16)).view(
        torch.bfloat16).to(device)
    kd = torch.from_numpy(oracle.fp8_dequant_rows(_codes_np(kc), ks_.cpu().numpy()).view(np.int16)).view(
        torch.bfloat16).to(device)
    ref = ops.indexer(qd, kd, w, None, k_top, True, 0, rope_dim=0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), exact.cpu().numpy())
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    # indices are a permutation prefix of the causal range per query
    g_np = got.cpu().numpy()[0]
    for s in (0, 5, 127):
        v = g_np[s][g_np[s] >= 0]
        assert len(set(v.tolist())) == len(v) and (v <= s).all()


# ------------------------------------------------------------------ the FP8 matrix instruction
def _e4m3(v):
    return int(oracle.e4m3_encode(np.float32(v)))


def _fp8_chain(rows_a, rows_b):
    """Run one v_mfma_scale_f32_16x16x128_f8f6f4 (unit scales) per case; row 0 of A against column 0 of B."""
    n = len(rows_a)
    A = np.zeros((n, 1, 16, 128), np.uint8)
    Bm = np.zeros_like(A)
    for t, (a, b) in enumerate(zip(rows_a, rows_b)):
        A[t, 0, 0] = a
        Bm[t, 0, 0] = b
    tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(Bm).cuda()
    tC = torch.zeros(n, 16, 16, dtype=torch.float32, device="cuda")
    tD = torch.empty_like(tC)
    _lib.check(_lib.load().ks_dbg_mfma_fp8_chain(tA.data_ptr(), tB.data_ptr(), tC.data_ptr(), tD.data_ptr(), n, 1,
                                                 torch.cuda.current_stream().cuda_stream), "fp8 chain")
    torch.cuda.synchronize()
    return tD.cpu().numpy()[:, 0, 0]


def test_fp8_mfma_alignment_window(device):
    # products (a_i b_i) of e4m3 operands in one instruction: [p, small, -p]; the exact sum is `small`
    def case(p, small):
        a = np.zeros(128, np.uint8)
        b = np.zeros(128, np.uint8)
        for i, (x, y) in enumerate([p, small, (p[0], -p[1])]):
            a[i], b[i] = _e4m3(x), _e4m3(y)
        return a, b
    cases = [
        case((-256.0, -1.0), (-16.0, -2.0 ** -9)),   # 2^8, 2^-5: kept
        case((-256.0, -1.0), (-8.0, -2.0 ** -9)),    # 2^8, 2^-6: dropped
        case((-256.0, -2.0 ** -8), (-2.0, -2.0 ** -9)),  # 1, 2^-8: kept
    ]
    print("[case] fp8 mfma alignment window", flush=True)
    got = _fp8_chain([c[0] for c in cases], [c[1] for c in cases])
    assert got[0] == 2.0 ** -5
    assert got[1] == 0.0          # exact: 2^-6; the instruction dropped it next to 2^8
    assert got[2] == 2.0 ** -8    # 1 + 2^-8 - 1 in range of the window
    # small integers are exact (no alignment loss): a layout check of the probe itself
    rng = np.random.default_rng(0)
    small = np.array([_e4m3(v) for v in (-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0)], np.uint8)
    a = rng.choice(small, (8, 128))
    b = rng.choice(small, (8, 128))
    got = _fp8_chain(list(a), list(b))
    want = (oracle.e4m3_decode(a).astype(np.float64) * oracle.e4m3_decode(b)).sum(1)
    np.testing.assert_array_equal(got, want)


def test_fp8_plain_mfma_alignment_window(device):
    # the plain instruction v_mfma_f32_16x16x32_fp8_fp8 (no block scales) aligns the products of one group of
    # eight k-slots to 13 bits below the group's largest, like the scaled one: with 2^8, small, -2^8 in slots 0, 1, 2
    # a small product of 2^-5 is kept and 2^-6 dropped.  Across groups (slots 0, 8, 16) the running value keeps far
    # more (2^-15 next to 2^8), so the window is per group of eight.  Small integers are exact in both layouts,
    # which also checks that the operands are read as OCP e4m3.
    def run(A, Bm):
        n = A.shape[0]
        tA, tB = torch.from_numpy(A).cuda(), torch.from_numpy(Bm).cuda()
        tC = torch.zeros(n, 16, 16, dtype=torch.float32, device="cuda")
        tD = torch.empty_like(tC)
        _lib.check(_lib.load().ks_dbg_mfma_fp8_plain_chain(tA.data_ptr(), tB.data_ptr(), tC.data_ptr(), tD.data_ptr(),
                                                           n, A.shape[1], torch.cuda.current_stream().cuda_stream),
                   "fp8 plain chain")
        torch.cuda.synchronize()
        return tD.cpu().numpy()

    def case(small, pos):
        a = np.zeros((1, 16, 32), np.uint8)
        b = np.zeros_like(a)
        for i, (x, y) in zip(pos, [(16.0, 16.0), small, (16.0, -16.0)]):
            a[0, 0, i], b[0, 0, i] = _e4m3(x), _e4m3(y)
        return a, b
    print("[case] plain fp8 mfma alignment window", flush=True)
    smalls = [(0.5, 2.0 ** -4), (0.25, 2.0 ** -4), (2.0 ** -6, 2.0 ** -9)]  # 2^-5, 2^-6, 2^-15
    cases = [case(sv, (0, 1, 2)) for sv in smalls] + [case(sv, (0, 8, 16)) for sv in smalls]
    got = run(np.stack([c[0] for c in cases]), np.stack([c[1] for c in cases]))[:, 0, 0]
    assert got[0] == 2.0 ** -5 and got[1] == 0.0 and got[2] == 0.0   # one group: 13 bits
    assert got[3] == 2.0 ** -5 and got[4] == 2.0 ** -6 and got[5] == 2.0 ** -15  # across groups
    rng = np.random.default_rng(0)
    small = np.array([_e4m3(v) for v in (-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0)], np.uint8)
    A = rng.choice(small, (8, 2, 16, 32)).astype(np.uint8)
    Bm = rng.choice(small, (8, 2, 16, 32)).astype(np.uint8)
    want = np.einsum("tcik,tcjk->tij", oracle.e4m3_decode(A).astype(np.float64), oracle.e4m3_decode(Bm))
    np.testing.assert_array_equal(run(A, Bm), want)


def test_fp8_hardware_conversions(device):
    # the conversions the bounded FP8 kernels use to dequantise codes in registers: v_cvt_pk_f32_fp8 gives every
    # code's value exactly; v_cvt_scalef32_pk_bf16_fp8 gives bf16(value * s) for a power-of-two s in [2^-100, 2^100]
    # and applies only the exponent of any other scale (its mantissa and sign are ignored)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    codes = torch.arange(256, dtype=torch.uint8, device=device)
    vals = oracle.e4m3_decode(np.arange(256, dtype=np.uint8))
    print("[case] fp8 hardware conversions", flush=True)
    out = torch.empty(256, dtype=torch.float32, device=device)
    _lib.check(lib.ks_dbg_fp8_cvt(codes.data_ptr(), 0, 256, 0, out.data_ptr(), st), "fp8 cvt")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    nan = np.isnan(vals)
    assert (np.isnan(got) == nan).all() and np.array_equal(got[~nan], vals[~nan])
    assert np.array_equal(got[~nan].view(np.uint32), vals[~nan].view(np.uint32))  # signed zeros too
    for s, exact in [(2.0 ** -100, True), (2.0 ** -22, True), (1.0, True), (2.0 ** 20, True), (2.0 ** 100, True),
                     (0.75, False), (3.0, False), (-2.0, False)]:
        sc = torch.full((256,), s, dtype=torch.float32, device=device)
        o = torch.empty(256, dtype=torch.int16, device=device)
        _lib.check(lib.ks_dbg_fp8_cvt(codes.data_ptr(), sc.data_ptr(), 256, 1, o.data_ptr(), st), "fp8 scaled cvt")
        torch.cuda.synchronize()
        g = o.cpu().numpy().view(np.uint16)[~nan]
        want = oracle.f32_to_bf16((vals * np.float32(s)).astype(np.float32))[~nan]
        if exact:
            np.testing.assert_array_equal(g, want)
        else:
            # only the exponent of |s| is applied
            e = np.float32(2.0 ** np.floor(np.log2(abs(s))))
            np.testing.assert_array_equal(g, oracle.f32_to_bf16((vals * e).astype(np.float32))[~nan])
            assert not np.array_equal(g, want)


@pytest.mark.parametrize("seed", [0, 1])
def test_indexer_fp8_bounded_arbitrary_scales(device, seed):
    # the bounded path (64 heads, D = 128, fp32 weights) reads the codes itself; rows whose scales are not powers of
    # two, or lie outside [2^-100, 2^100], take the exact multiply-and-round conversion, the others the one-instruction
    # form, mixed within waves and key blocks; indices bit-exact against the oracle on the dequantised rows
    g = torch.Generator().manual_seed(40 + seed)
    B, S, H, D, T, k_top = 1, 24, 64, 128, 1500, 256
    rng = np.random.default_rng(seed)
    def codes(shape):
        c = rng.integers(0, 256, shape).astype(np.uint8)
        c[(c & 0x7F) == 0x7F] = 0x3C  # no NaN codes
        return c
    def scales(shape):
        kind = rng.integers(0, 4, shape)
        s = np.where(kind == 0, 2.0 ** rng.integers(-12, 4, shape),                  # power of two: one instruction
            np.where(kind == 1, rng.uniform(0.01, 2.0, shape),                         # arbitrary fp32 scale
            np.where(kind == 2, 2.0 ** rng.integers(-112, -101, shape),               # power of two below the range
                     2.0 ** rng.integers(-8, 2, shape) * 1.5)))                        # mantissa bit set
        return s.astype(np.float32)
    qc, kc = codes((B, S, H, D)), codes((B, T, D))
    if seed == 1:  # whole waves and key blocks of each form as well
        qs = np.full((B, S, H), 0.0625, np.float32)
        qs[:, S // 2:] = scales((B, S - S // 2, H))
        ks_ = np.full((B, T), 0.125, np.float32)
        ks_[:, 512:1024] = scales((B, 512))
    else:
        qs, ks_ = scales((B, S, H)), scales((B, T))
    w = torch.randn(B, S, H, generator=g) / 8
    print(f"[case] indexer fp8 bounded arbitrary scales seed={seed}", flush=True)
    out = ops.indexer_fp8(torch.from_numpy(qc).to(device), torch.from_numpy(qs).to(device),
                          torch.from_numpy(kc).to(device), torch.from_numpy(ks_).to(device), w.to(device), k_top,
                          True, T - S)
    torch.cuda.synchronize()
    want = oracle.indexer_fp8(qc, qs, kc, ks_, w.numpy(), k_top, True, T - S)
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
