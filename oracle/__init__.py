"""CPU oracle for the three KernelSwift operators — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
package, and only as the checker (or, for bench, as the timed CPU baseline); the
product path (kernelswift_amd) never imports it.

Each function restates the reference algorithm in plain numpy (fp64 where the
reference computes in floating point with a tolerance contract) or, for the
bit-exact indexer path, in the canonical arithmetic order implemented by the C
library ks_oracle.c.  Citations are to /root/reference files.

Pinning (what checks each function beyond restating it; see tests/test_oracle.py):
  sinkhorn        closed forms (constant input -> 1/4), doubly-stochastic invariant,
                  permutation equivariance, fp64-vs-fp32 restatements agree.
  rope_bf16       identity at position 0, unit vectors -> (cos, sin), inverse
                  rotation composes to ~identity, complex128 multiply agrees.
  dot_exact       exact rational arithmetic (fractions.Fraction) on random and
                  adversarial vectors (cancellation, subnormals, ties at midpoints).
  indexer_scores  single-head case reduces to relu(dot)*w, brute-force Fraction
                  recomputation of the canonical order on tiny shapes, mask closed form.
  topk_stable     brute force over all permutations of tiny rows, ties and -inf.
  postprocess     integer closed form of baseline/indexer.py:198-206.
  e4m3_encode     torch's float8_e4m3fn conversion (a library routine) over every bf16
                  value in range and every tie midpoint, and nearest-value brute force.
  e4m3_decode     torch's float8_e4m3fn -> float32 over all 256 codes.
  fp8_quant_rows  closed forms (ue8m0 scales are powers of two with amax/s in (224, 448];
                  the largest element maps to a code of the top binade; all-zero rows
                  take the 1e-4 floor), torch's cast of the scaled rows.
  sparse_attn     closed forms: all-invalid -> 0; equal scores -> k/(k+e^(sink-z)) *
                  mean(V); single valid index with sink -> -inf gives that V row;
                  duplicates counted with multiplicity.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libks_oracle.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build as _b  # noqa: F401  (relative import of oracle/build.py)
            _b.build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.ko_dot_exact_bf16.restype = ctypes.c_uint16
        lib.ko_dot_exact_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.ko_dot_matrix.restype = None
        lib.ko_dot_matrix.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_int]
        lib.ko_indexer_scores.restype = None
        lib.ko_indexer_scores.argtypes = ([ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p]
                                          + [ctypes.c_int64] * 6 + [ctypes.c_int, ctypes.c_int64,
                                                                    ctypes.c_int, ctypes.c_int])
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def default_threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:  # pragma: no cover
        return max(1, min(16, os.cpu_count() or 1))


# ---------------------------------------------------------------- bf16 helpers
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """Raw bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


# ---------------------------------------------------------------- Sinkhorn
def sinkhorn(x: np.ndarray, repeat: int = 10, eps: float = 1e-6) -> np.ndarray:
    """fp64 restatement of baseline/sinkhorn.py:13-19 over the last two axes.

    softmax over the last axis (no eps in its denominator), + eps, then a column
    normalisation (sum over axis -2), then repeat-1 x (row, column) normalisations,
    each dividing by (sum + eps).
    """
    v = np.asarray(x, dtype=np.float64)
    v = v - v.max(axis=-1, keepdims=True)
    v = np.exp(v)
    v = v / v.sum(axis=-1, keepdims=True) + eps
    v = v / (v.sum(axis=-2, keepdims=True) + eps)
    for _ in range(repeat - 1):
        v = v / (v.sum(axis=-1, keepdims=True) + eps)
        v = v / (v.sum(axis=-2, keepdims=True) + eps)
    return v


# ---------------------------------------------------------------- RoPE
def freqs_table(rope_dim: int, n_pos: int, theta: float = 10000.0) -> np.ndarray:
    """(cos, sin) table [n_pos, rope_dim/2, 2] float32 of baseline/indexer.py:226-235.

    Computed with torch on the CPU exactly as the reference builds freqs_cis
    (fp32 freqs, fp32 outer product, torch.polar), then viewed as real pairs.
    The kernels and this oracle both consume the table as an input.
    """
    import torch
    freqs = 1.0 / (theta ** (torch.arange(0, rope_dim, 2).float() / rope_dim))
    pos = torch.arange(n_pos, dtype=torch.float32)
    ang = torch.outer(pos, freqs)
    cis = torch.polar(torch.ones_like(ang), ang)
    return torch.view_as_real(cis).contiguous().numpy()


def rope_bf16(x: np.ndarray, freqs: np.ndarray, rope_start: int, rope_dim: int, pos0: int = 0) -> np.ndarray:
    """Canonical RoPE on bf16 rows x [B, S, H, D] (uint16), returning a new array.

    apply_rotary_emb (baseline/indexer.py:114-129): pairs (2j, 2j+1) of the segment
    [rope_start, rope_start+rope_dim) times (cos, sin) of position pos0+s, fp32
    math with separately rounded products (numpy float32 ops never fuse), RNE back
    to bf16 (the .copy_ into the bf16 tensor, :128).
    """
    x = np.array(x, dtype=np.uint16, copy=True)
    B, S, H, D = x.shape
    seg = bf16_to_f32(x[..., rope_start:rope_start + rope_dim]).reshape(B, S, H, rope_dim // 2, 2)
    cs = freqs[pos0:pos0 + S].astype(np.float32)  # [S, P, 2]
    c = cs[None, :, None, :, 0]
    s = cs[None, :, None, :, 1]
    x0 = seg[..., 0]
    x1 = seg[..., 1]
    y0 = (x0 * c) - (x1 * s)
    y1 = (x0 * s) + (x1 * c)
    out = np.stack([y0, y1], axis=-1).reshape(B, S, H, rope_dim).astype(np.float32)
    x[..., rope_start:rope_start + rope_dim] = f32_to_bf16(out)
    return x


# ---------------------------------------------------------------- exact dots / scores
def dot_exact(a: np.ndarray, b: np.ndarray) -> int:
    """bf16 bits of the exact dot of two bf16 vectors, rounded once (RNE)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    assert a.shape == b.shape and a.ndim == 1
    return int(_load().ko_dot_exact_bf16(_ptr(a), _ptr(b), a.shape[0]))


def dot_matrix(A: np.ndarray, B: np.ndarray, threads: Optional[int] = None) -> np.ndarray:
    """bf16 bits [M, N] of exact dots of rows of A [M, D] with rows of B [N, D]."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    B = np.ascontiguousarray(B, dtype=np.uint16)
    M, D = A.shape
    N = B.shape[0]
    out = np.empty((M, N), dtype=np.uint16)
    _load().ko_dot_matrix(_ptr(A), _ptr(B), _ptr(out), M, N, D, threads or default_threads())
    return out


def indexer_scores(q: np.ndarray, k: np.ndarray, w: np.ndarray, causal: bool, start_pos: int, ratio: int = 1,
                   T: Optional[int] = None, threads: Optional[int] = None) -> np.ndarray:
    """Canonical scores [B, S, T] float32 (see ks_oracle.c for the order).

    q: bf16 bits [B, S, H, D]; k: bf16 bits [B, Tk, D] (first T rows used);
    w: float32 [B, S, H] (fp32 weights) or uint16 bf16 bits (bf16 weights).
    """
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    B, S, H, D = q.shape
    Tk = k.shape[1]
    T = Tk if T is None else T
    w_bf16 = 1 if w.dtype == np.uint16 else 0
    w = np.ascontiguousarray(w, dtype=np.uint16 if w_bf16 else np.float32)
    assert k.shape[0] == B and k.shape[2] == D and w.shape == (B, S, H) and T <= Tk
    out = np.empty((B, S, T), dtype=np.float32)
    _load().ko_indexer_scores(_ptr(q), _ptr(k), _ptr(w), w_bf16, _ptr(out), B, S, H, D, T, Tk,
                              1 if causal else 0, start_pos, ratio, threads or default_threads())
    return out


# ---------------------------------------------------------------- TopK
def topk_stable(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices [..., k] (int64) of a stable descending sort's prefix over the last axis.

    This is the tie contract of the reference TopK (equal scores, -inf included, keep
    ascending column order; optimized/indexer_project/design.md:99-105) applied to
    index_score.topk(k) (baseline/indexer.py:195-196).  Library routine:
    numpy's stable mergesort on negated keys.
    """
    s = np.asarray(scores, dtype=np.float32)
    assert not np.isnan(s).any(), "NaN scores are outside the contract"
    order = np.argsort(-s, axis=-1, kind="stable")
    return order[..., :k].astype(np.int64)


def postprocess(idx: np.ndarray, causal: bool, start_pos: int, ratio: int, offset: int) -> np.ndarray:
    """baseline/indexer.py:198-206, generalised to any start_pos when causal.

    idx [B, S, k] int64; query s has limit (start_pos+s+1)//ratio; causal: idx >= limit
    -> -1 else idx+offset; non-causal: idx+offset.
    """
    idx = np.asarray(idx, dtype=np.int64)
    if not causal:
        return idx + offset
    S = idx.shape[-2]
    lim = (start_pos + np.arange(S, dtype=np.int64) + 1) // ratio
    return np.where(idx >= lim[:, None], -1, idx + offset)


def indexer(q: np.ndarray, k: np.ndarray, w: np.ndarray, freqs: np.ndarray, k_top: int, causal: bool,
            start_pos: int, ratio: int = 1, offset: int = 0, rope_start: int = 0, rope_dim: int = 64,
            rope_k: bool = True, threads: Optional[int] = None) -> np.ndarray:
    """Full indexer path: RoPE(q at positions start_pos+s, k at t) -> canonical scores ->
    stable top-k -> post-processing.  Returns int64 [B, S, min(k_top, T)]."""
    B, S, H, D = q.shape
    T = k.shape[1]
    qr = rope_bf16(q, freqs, rope_start, rope_dim, pos0=start_pos)
    kr = k
    if rope_k:
        kr = rope_bf16(k.reshape(B, T, 1, D), freqs, rope_start, rope_dim, pos0=0).reshape(B, T, D)
    sc = indexer_scores(qr, kr, w, causal, start_pos, ratio, threads=threads)
    kk = min(k_top, T)
    return postprocess(topk_stable(sc, kk), causal, start_pos, ratio, offset)


# ---------------------------------------------------------------- FP8 (e4m3fn) rows
# The reference names an FP8 configuration of its DeepSeek-style model (dtype = "fp8", scale_fmt = "ue8m0";
# baseline/indexer.py:14-17) but ships no kernel for it; these functions state the quantised indexer that the
# library implements: block quantisation to e4m3fn with per-block fp32 scales, and the indexer run on the
# dequantised rows (the scoring of baseline/indexer.py:191-206 without RoPE, which precedes quantisation).
_INV448 = np.float32(1.0) / np.float32(448.0)


def e4m3_encode(y) -> np.ndarray:
    """e4m3fn codes (uint8) of float32 values with |y| <= 448, rounded to nearest even (ties to the even
    code); -0 and negative values that round to zero keep the sign bit."""
    y = np.asarray(y, dtype=np.float32)
    sign = ((y.view(np.uint32) >> 24) & 0x80).astype(np.int64)
    a = np.abs(y).astype(np.float64)
    _, ex = np.frexp(a)  # a = m 2^ex, 0.5 <= m < 1: the exponent of a is ex - 1
    e = ex.astype(np.int64) - 1
    sub = a < 2.0 ** -6
    q_sub = np.rint(a * 512.0).astype(np.int64)            # multiples of 2^-9 (q = 8 is 2^-6 itself)
    es = np.where(sub, 0, e)
    q_nrm = np.rint(np.ldexp(a, 3 - es)).astype(np.int64)  # a / 2^(e-3) in [8, 16]; 16 carries
    code = np.where(sub, q_sub, ((es + 7) << 3) + q_nrm - 8)
    return (sign | code).astype(np.uint8)


def e4m3_decode(c) -> np.ndarray:
    """Values (float32, exact) of e4m3fn codes; the NaN codes 0x7F / 0xFF give NaN."""
    c = np.asarray(c, dtype=np.uint8).astype(np.int64)
    e = (c >> 3) & 15
    m = c & 7
    a = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.ldexp(1.0, e - 10))
    a = np.where((c & 0x7F) == 0x7F, np.nan, a)
    return np.where(c & 0x80, -a, a).astype(np.float32)


def fp8_quant_rows(x: np.ndarray, block: int, ue8m0: bool = True):
    """Block quantisation of bf16 rows: per block of `block` elements of the last dim,
    amax = max(max|x|, fp32(1e-4)), s = fp32(amax * fp32(1/448)), under ue8m0 s = 2^ceil(log2 s), and
    code = e4m3fn(clip(fp32(x / s), -448, 448)).  x: bf16 bits [..., D].
    Returns (codes uint8 [..., D], scales float32 [..., D / block])."""
    x = np.asarray(x, dtype=np.uint16)
    D = x.shape[-1]
    assert D % block == 0
    xf = bf16_to_f32(x).reshape(*x.shape[:-1], D // block, block)
    amax = np.maximum(np.abs(xf).max(axis=-1), np.float32(1e-4)).astype(np.float32)
    s = (amax * _INV448).astype(np.float32)
    if ue8m0:
        m, ex = np.frexp(s.astype(np.float64))   # s = m 2^ex: ceil(log2 s) = ex - 1 when m == 1/2, else ex
        s = np.ldexp(1.0, np.where(m == 0.5, ex - 1, ex)).astype(np.float32)
    y = np.clip((xf / s[..., None]).astype(np.float32), np.float32(-448.0), np.float32(448.0))
    return e4m3_encode(y).reshape(x.shape), s


def fp8_dequant_rows(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """bf16 bits of bf16(fp32(value(code) * scale)) with one scale per row (scales: codes.shape[:-1])."""
    v = e4m3_decode(codes) * np.asarray(scales, dtype=np.float32)[..., None]
    return f32_to_bf16(v.astype(np.float32))


def indexer_fp8(qc: np.ndarray, qs: np.ndarray, kc: np.ndarray, ks: np.ndarray, w: np.ndarray, k_top: int,
                causal: bool, start_pos: int, ratio: int = 1, offset: int = 0,
                threads: Optional[int] = None) -> np.ndarray:
    """Indexer on FP8 rows: canonical scores of the dequantised q [B, S, H, D] and k [B, T, D] (one scale
    per row: qs [B, S, H], ks [B, T]) -> stable top-k -> post-processing.  Returns int64 [B, S, min(k_top, T)]."""
    q = fp8_dequant_rows(qc, qs)
    k = fp8_dequant_rows(kc, ks)
    sc = indexer_scores(q, k, w, causal, start_pos, ratio, threads=threads)
    kk = min(k_top, k.shape[1])
    return postprocess(topk_stable(sc, kk), causal, start_pos, ratio, offset)


# ---------------------------------------------------------------- sparse attention
def sparse_attn(q: np.ndarray, kv: np.ndarray, sink: np.ndarray, idx: np.ndarray, scale: float,
                dv: Optional[int] = None) -> np.ndarray:
    """fp64 restatement of sparse_attn_ref (baseline/sparse_attention.py:5-42).

    q: bf16 bits [B, M, H, Dqk]; kv: bf16 bits [B, N, Dqk]; sink float32 [H];
    idx int32 [B, M, K] (negative = invalid).  V = kv[..., :dv].  Returns float64
    [B, M, H, dv] (before the final bf16 cast of the reference).
    """
    B, M, H, Dqk = q.shape
    dv = Dqk if dv is None else dv
    qf = bf16_to_f32(q).astype(np.float64)
    kvf = bf16_to_f32(kv).astype(np.float64)
    idx = np.asarray(idx)
    valid = idx >= 0
    safe = np.where(valid, idx, 0).astype(np.int64)
    out = np.empty((B, M, H, dv), dtype=np.float64)
    sink64 = np.asarray(sink, dtype=np.float64)
    for b in range(B):
        g = kvf[b][safe[b]]                     # [M, K, Dqk]  (gather, :16-22)
        g = np.where(valid[b][..., None], g, 0.0)
        s = np.einsum("mhd,mtd->mht", qf[b], g) * scale          # (:24-27)
        s = np.where(valid[b][:, None, :], s, -np.inf)
        z = np.maximum(s.max(axis=-1, keepdims=True), sink64[None, :, None])  # (:29-31)
        e = np.where(valid[b][:, None, :], np.exp(s - z), 0.0)
        den = e.sum(axis=-1, keepdims=True) + np.exp(sink64[None, :, None] - z)
        p = e / den
        out[b] = np.einsum("mht,mtd->mhd", p, g[..., :dv])      # (:39-41)
    return out


# ---------------------------------------------------------------- mHC hyper-connections
def _sigmoid(z: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-z))


def mhc_pre(x: np.ndarray, pre_logits: np.ndarray) -> np.ndarray:
    """Layer input of an mHC block (hc_mult = 4; baseline/indexer.py:48-50 configures the connections):
    h[t] = sum_j sigmoid(pre_logits[t, j]) x[t, j].  x: bf16 bits [N, 4, C]; returns float64 [N, C]."""
    xf = bf16_to_f32(x).astype(np.float64)
    g = _sigmoid(np.asarray(pre_logits, np.float64))
    return np.einsum("nj,njc->nc", g, xf)


def mhc_post(x: np.ndarray, f: np.ndarray, res_logits: np.ndarray, post_logits: np.ndarray,
             sinkhorn_iters: int = 20, eps: float = 1e-6) -> np.ndarray:
    """Residual update of an mHC block: out[t, i] = sum_j S[t, i, j] x[t, j] + 2 sigmoid(post_logits[t, i]) f[t],
    S = sinkhorn(res_logits, repeat=sinkhorn_iters, eps) (baseline/sinkhorn.py:13-19, in fp64 above).
    x: bf16 bits [N, 4, C]; f: bf16 bits [N, C]; returns float64 [N, 4, C]."""
    xf = bf16_to_f32(x).astype(np.float64)
    ff = bf16_to_f32(f).astype(np.float64)
    S = sinkhorn(np.asarray(res_logits, np.float32), sinkhorn_iters, eps).astype(np.float64)
    p = 2.0 * _sigmoid(np.asarray(post_logits, np.float64))
    return np.einsum("nij,njc->nic", S, xf) + p[:, :, None] * ff[:, None, :]
