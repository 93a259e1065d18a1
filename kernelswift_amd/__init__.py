"""KernelSwift operators for AMD Instinct MI355X (gfx950).

Three fused operators, each a hand-written HIP kernel set behind the C ABI of
include/kswift.h (libkswift_amd.so), with torch-facing wrappers in ``ops`` and
drop-in ``ModelNew`` modules in ``optimized``:

* Sinkhorn normalisation of 4x4 matrices          -> ops.sinkhorn
* DeepSeek-style indexer (RoPE, exact scores, exact top-k) -> ops.indexer, ops.indexer_scores, ops.topk_mask
* top-k sparse attention with an attention sink   -> ops.sparse_attn
"""
from . import ops  # noqa: F401

__version__ = "0.1.0"
