"""CPU checks of the C-ABI boundary: the library loads, exports every entry point include/kswift.h
declares (no compute calls without a GPU), and host-side argument validation fails loudly."""
import ctypes
import os
import re

import pytest

from kernelswift_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "kswift.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"\b(ks_[a-z0-9_]+)\s*\(", src)


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.ks_version() == 100


def test_host_validation_without_gpu():
    lib = _lib.load()
    # invalid arguments are rejected on the host before any HIP call
    assert lib.ks_sinkhorn(None, None, 5, 0, 1e-6, None) == 1
    assert b"repeat" in lib.ks_last_error()
    assert lib.ks_sinkhorn(None, None, 0, 1, 1e-6, None) == 0  # empty batch is a no-op
    assert lib.ks_indexer_topk(None, 10, 1, 1, 10, 11, 0, 0, 1, 0, None, 0, None) == 1
    assert b"k=" in lib.ks_last_error()
    assert lib.ks_sparse_attn(None, None, None, None, None, 1, 1, 16, 64, 64, 8, 4, 0.1, None, 0, None) == 1
    assert b"supported" in lib.ks_last_error()
    assert lib.ks_indexer_scores(None, None, None, 0, None, None, None, None, None, 1, 1, 64, 96, 10, 10, 0, 0, 1,
                                 None) == 1
    assert lib.ks_rope_inplace(None, None, 1, 1, 1, 128, 4, 64, 0, 10, None) == 1


def test_workspace_queries():
    lib = _lib.load()
    assert lib.ks_indexer_workspace_size(1, 128, 64, 128, 4096) >= 128 * 4096 * 4  # the fp32 score matrix
    # many queries -> one range per query -> no workspace
    assert lib.ks_sparse_attn_workspace_size(8, 2600, 64, 128, 128, 16) == 0
    assert lib.ks_sparse_attn_workspace_size(32, 1, 128, 576, 512, 2048) > 0


def test_ops_refuse_cpu_tensors():
    import torch
    from kernelswift_amd import ops
    with pytest.raises(RuntimeError):
        ops.sinkhorn(torch.zeros(2, 4, 4))
    with pytest.raises(RuntimeError):
        ops.sparse_attn(torch.zeros(1, 1, 16, 128, dtype=torch.bfloat16), torch.zeros(1, 4, 128, dtype=torch.bfloat16),
                        torch.zeros(16), torch.zeros(1, 1, 2, dtype=torch.int32), 0.1)
