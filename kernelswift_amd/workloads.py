"""Synthetic inputs for the five BASELINE.json configurations (seeded, deterministic).

Order of generation follows the configuration text: torch.manual_seed(seed), then each tensor in the
listed order on the CPU, then moved to the device.  The only exception is config 5's 2.25 GiB kv cache,
which is drawn on the device itself with a seeded device generator (a CPU draw of 1.2 G normals would
dominate every run); its gathered rows are copied back when a CPU check needs them.

Configs (BASELINE.json "configs"):
  1 sinkhorn         x [16384, 4, 4] fp32 N(0,1); repeat 10 (20 normalisations), eps 1e-6
  2 indexer_short    q [1,128,64,128] bf16, k [1,4096,128] bf16, w [1,128,64] fp32 N(0,1)/8, RoPE on dims
                     0..63 (theta 1e4) of q (positions start_pos+i) and k (positions t), causal with
                     start_pos = S_kv - S_q, top-512
  3 sparse_prefill   q [1,128,16,128] bf16, kv [1,8192,128] bf16, query i at position 8064+i takes
                     randperm(pos+1)[:2048] int32, sink zeros(16), scale 128^-0.5
  4 indexer_long     as 2 with S_q = 64, S_kv = 32768, top-2048
  5 mla_decode       q [32,1,128,576] bf16, kv [32,65536,576] bf16, idx = randperm(65536)[:2048] per
                     sequence, sink zeros(128), scale 576^-0.5, dv = 512
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict

import torch

SEED = 42


def freqs_table(rope_dim: int, n_pos: int, theta: float = 10000.0) -> torch.Tensor:
    """(cos, sin) float32 [n_pos, rope_dim/2, 2]: the real view of freqs_cis built as in
    baseline/indexer.py:226-235 (fp32 inverse frequencies, fp32 outer product, polar)."""
    freqs = 1.0 / (theta ** (torch.arange(0, rope_dim, 2).float() / rope_dim))
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float32), freqs)
    return torch.view_as_real(torch.polar(torch.ones_like(ang), ang)).contiguous()


@dataclass
class Workload:
    name: str
    op: str
    tensors: Dict[str, torch.Tensor]
    params: Dict[str, object] = field(default_factory=dict)


def sinkhorn_cfg(device="cpu", seed=SEED, n=16384, repeat=10) -> Workload:
    torch.manual_seed(seed)
    x = torch.randn(n, 4, 4, dtype=torch.float32)
    return Workload("sinkhorn", "sinkhorn", {"x": x.to(device)}, {"repeat": repeat, "eps": 1e-6})


def indexer_cfg(device="cpu", seed=SEED, S=128, T=4096, H=64, D=128, k_top=512) -> Workload:
    torch.manual_seed(seed)
    q = torch.randn(1, S, H, D).to(torch.bfloat16)
    k = torch.randn(1, T, D).to(torch.bfloat16)
    w = torch.randn(1, S, H, dtype=torch.float32) / 8
    freqs = freqs_table(64, T)
    return Workload(f"indexer_S{S}_T{T}", "indexer",
                    {"q": q.to(device), "k": k.to(device), "w": w.to(device), "freqs": freqs.to(device)},
                    {"k_top": k_top, "causal": True, "start_pos": T - S, "ratio": 1, "offset": 0, "rope_start": 0,
                     "rope_dim": 64, "rope_k": True})


def sparse_prefill_cfg(device="cpu", seed=SEED, S=128, H=16, D=128, N=8192, K=2048) -> Workload:
    torch.manual_seed(seed)
    q = torch.randn(1, S, H, D).to(torch.bfloat16)
    kv = torch.randn(1, N, D).to(torch.bfloat16)
    start = N - S
    g = torch.Generator().manual_seed(seed)
    idx = torch.empty(1, S, K, dtype=torch.int32)
    for i in range(S):
        pos = start + i
        idx[0, i] = torch.randperm(pos + 1, generator=g)[:K].to(torch.int32)
    sink = torch.zeros(H, dtype=torch.float32)
    return Workload("sparse_prefill", "sparse_attn",
                    {"q": q.to(device), "kv": kv.to(device), "idx": idx.to(device), "sink": sink.to(device)},
                    {"scale": D ** -0.5, "dv": D})


def mla_decode_cfg(device="cpu", seed=SEED, B=32, H=128, Dqk=576, Dv=512, N=65536, K=2048) -> Workload:
    torch.manual_seed(seed)
    q = torch.randn(B, 1, H, Dqk).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)]).to(torch.int32).view(B, 1, K)
    sink = torch.zeros(H, dtype=torch.float32)
    dev = torch.device(device)
    if dev.type == "cuda":
        dg = torch.Generator(device=dev).manual_seed(seed)
        kv = torch.empty(B, N, Dqk, dtype=torch.bfloat16, device=dev)
        for b in range(B):  # per-sequence draws keep the fp32 temporary at 151 MB
            kv[b] = torch.randn(N, Dqk, generator=dg, device=dev).to(torch.bfloat16)
    else:
        kv = torch.randn(B, N, Dqk).to(torch.bfloat16)
    return Workload("mla_decode", "sparse_attn",
                    {"q": q.to(device), "kv": kv, "idx": idx.to(device), "sink": sink.to(device)},
                    {"scale": Dqk ** -0.5, "dv": Dv})


CONFIGS = {
    1: lambda device="cpu": sinkhorn_cfg(device),
    2: lambda device="cpu": indexer_cfg(device, S=128, T=4096, k_top=512),
    3: lambda device="cpu": sparse_prefill_cfg(device),
    4: lambda device="cpu": indexer_cfg(device, S=64, T=32768, k_top=2048),
    5: lambda device="cpu": mla_decode_cfg(device),
}

# Algorithmic work per call (basis of the roofline fractions): bytes for HBM-bound ops, flops for MFMA.
def algorithmic_work(cfg: int) -> Dict[str, float]:
    if cfg == 1:
        return {"bytes": 2 * 16384 * 16 * 4}
    if cfg in (2, 4):
        S, T = (128, 4096) if cfg == 2 else (64, 32768)
        return {"flops": 2.0 * S * 64 * T * 128, "bytes": S * 64 * 128 * 2 + T * 128 * 2 + S * 64 * 4}
    if cfg == 3:
        return {"flops": 2.0 * 128 * 16 * 2048 * (128 + 128), "gathered_bytes": 128 * 2048 * 256}
    if cfg == 5:
        return {"flops": 2.0 * 32 * 128 * 2048 * (576 + 512), "gathered_bytes": 32 * 2048 * 1152}
    raise KeyError(cfg)


def bf16_bits(t: torch.Tensor):
    """bf16 tensor -> numpy uint16 bit patterns (CPU copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")
