"""Writes tests/golden/mfma_bf16_gfx950.npz: operands and hardware results of chained
v_mfma_f32_16x16x32_bf16 instructions (ks_dbg_mfma_bf16_chain), so that the CPU suite can check the
accumulation model of tests/mfma_model.py against what the GPU computed.  Run on the GPU box:

    python tests/golden/make_mfma_fixture.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from tests import test_gpu_mfma_model as T  # noqa: E402

N = 96  # cases per set


def main() -> None:
    dev = torch.device("cuda:0")
    out = {}
    for name, (cases, nchain) in T.random_sets(np.random.default_rng(2024), N).items():
        hw = np.array(T._run(cases, nchain, dev), np.float32)
        out[name + "_a"] = np.stack([np.asarray(c[0], np.uint16).reshape(nchain, 32) for c in cases])
        out[name + "_b"] = np.stack([np.asarray(c[1], np.uint16).reshape(nchain, 32) for c in cases])
        out[name + "_c"] = np.array([c[2] for c in cases], np.float32)
        out[name + "_hw"] = hw
        print(name, len(cases), flush=True)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mfma_bf16_gfx950.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    main()
