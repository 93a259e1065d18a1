"""Drop-in modules on the CPU: importable without the GPU library (lazy loading), baseline parameter and
buffer names, reference ModelArgs duck typing, and loud failure instead of a CPU fallback."""
import importlib.util
import os

import pytest
import torch

from kernelswift_amd.optimized import indexer as ix
from kernelswift_amd.optimized import sinkhorn as sk
from kernelswift_amd.optimized import sparse_attention as sa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_state_dict_names_match_baseline():
    m = ix.ModelNew(*ix.get_init_inputs())
    assert sorted(m.state_dict().keys()) == ["freqs_cis", "kv_cache", "weights_proj.weight", "wq_b.weight"]
    assert m.wq_b.weight.shape == (16 * 64, 256) and m.wq_b.weight.dtype == torch.bfloat16
    assert m.weights_proj.weight.shape == (16, 1024)
    s = sa.ModelNew(*sa.get_init_inputs())
    assert list(s.state_dict().keys()) == ["attn_sink"] and s.softmax_scale == 128 ** -0.5


def test_load_state_dict_roundtrip():
    a = ix.ModelNew(*ix.get_init_inputs())
    b = ix.ModelNew(*ix.get_init_inputs())
    b.load_state_dict(a.state_dict())
    assert torch.equal(a.wq_b.weight, b.wq_b.weight) and torch.equal(a.kv_cache, b.kv_cache)


def test_freqs_real_view_accepted():
    args, fc, kv, r = ix.get_init_inputs()
    m1 = ix.ModelNew(args, fc, kv, r)
    m2 = ix.ModelNew(args, torch.view_as_real(fc), kv, r)
    assert torch.equal(m1._freqs(), m2._freqs()) and m1._freqs().shape == (2600, 16, 2)


def test_modules_load_by_path_without_library():
    # the reference harness loads v1 files by path; loading must not touch the GPU library
    for name in ("sinkhorn", "indexer", "sparse_attention"):
        path = os.path.join(ROOT, "kernelswift_amd", "optimized", f"{name}.py")
        spec = importlib.util.spec_from_file_location(f"v1_{name}", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        assert hasattr(mod, "ModelNew") and callable(mod.get_inputs) and callable(mod.get_init_inputs)


def test_cpu_tensors_fail_loudly():
    with pytest.raises(RuntimeError):
        sk.ModelNew()(torch.randn(1, 8, 4, 4))
