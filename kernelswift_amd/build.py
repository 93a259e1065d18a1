"""Build libkswift_amd.so (gfx950 HIP kernels + the C ABI of include/kswift.h) and
libkswift_torch.so (the TORCH_LIBRARY(ks_mi355x, ...) operator registration over that C ABI).

    python -m kernelswift_amd.build [-v]

Each csrc/*.hip is compiled to an object with hipcc for gfx950, then linked into
one shared library next to this file; csrc/torch_ops.cpp (host code only) is compiled
against the installed PyTorch-ROCm headers and linked to it.  Flags:
  -ffp-contract=off      no implicit FMA contraction: every fused multiply-add in
                         the kernels is an explicit __builtin_fmaf, so the bit-exact
                         indexer contract cannot be broken by the compiler;
  -packed-fp32-ops off   packed fp32 VALU forms are disabled (known-bad on this pool).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libkswift_amd.so")
TORCH_LIB = os.path.join(HERE, "libkswift_torch.so")
OBJ_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

# Per-file flags.  sparse_attn.hip: MFMA builtins in their VGPR form (accumulators in VGPRs).  The count-mask kernel
# rescales its O accumulators in a rarely taken branch; with AGPR accumulators the compiler moved all 64 of them
# to VGPRs and back on every chunk.  The file's other kernels keep AGPR accumulators through inline assembly
# (MLA) or fit in VGPRs either way.
FILE_FLAGS = {"sparse_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def flags(src: str) -> list:
    """hipcc flags of one source file (the common set plus its own)."""
    return [*COMMON, *FILE_FLAGS.get(os.path.basename(src), [])]


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *flags(src), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature; drop that harmless warning
    noise = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and "not a recognized feature" not in ln
             and ln.strip() != "1 warning generated."]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise))
    return obj


def build_torch_ops(verbose: bool = False) -> str:
    """The torch operator library: host C++ over the C ABI, so g++ suffices (no device code)."""
    import torch
    from torch.utils import cpp_extension
    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations"]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()] + ["-I/opt/rocm/include"]
    cmd += [os.path.join(CSRC, "torch_ops.cpp"), f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
            "-ltorch_hip", f"-L{HERE}", "-lkswift_amd", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}",
            "-o", TORCH_LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("g++ failed for torch_ops.cpp:\n" + r.stderr[-4000:])
    os.replace(TORCH_LIB + ".tmp", TORCH_LIB)
    return TORCH_LIB


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
