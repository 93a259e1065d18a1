"""No kernel of the library reads the AQL dispatch packet or uses flat memory instructions (CPU: hipcc
cross-compiles every source).

The dispatch packet lives in the HSA queue's ring buffer in host memory, so a kernel that needs it (for the
workgroup size: the compiler asks for it when it moves a per-thread array into LDS and must compute the flat
thread id) makes each workgroup's first scalar load a round trip to the host: one such array in the bounded
top-k's recomputation delayed every workgroup's first loads by 5-10 us.  The kernel descriptors record the
request as .amdhsa_user_sgpr_dispatch_ptr; this compiles each source with the library's flags and checks that
no kernel sets it.

Flat loads and stores count in lgkmcnt as well as vmcnt, so every wait for an LDS read (lgkmcnt(0) before an
LDS-fed MFMA) also waits for them: one pointer rebuilt from an integer, which the compiler treats as generic,
turned a sparse-attention kernel's index prefetch into flat loads that stalled each chunk's LDS reads.  The
same compile checks that no kernel contains a flat memory instruction."""
import concurrent.futures
import glob
import os
import re
import shutil
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def dispatch_ptr_kernels(asm: str):
    """Names of the kernels whose descriptor requests the dispatch pointer."""
    out = []
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", asm, re.S):
        d = re.search(r"\.amdhsa_user_sgpr_dispatch_ptr\s+(\d+)", m.group(2))
        if d is not None and d.group(1) != "0":
            out.append(m.group(1))
    return out


def flat_memory_kernels(asm: str):
    """Names of the kernels (entry points with a kernel descriptor) whose own code contains a flat load, store
    or atomic.  Non-inlined device functions are not checked: their pointer parameters are generic by nature,
    and the library calls them only on rare paths (the integer-accumulator exact dot, the merge-sort fallback)."""
    kernels = set(re.findall(r"\.amdhsa_kernel (\S+)", asm))
    out = []
    for m in re.finditer(r"^(\w+):[^\n]*\n(.*?)^\.Lfunc_end", asm, re.S | re.M):
        if m.group(1) in kernels and re.search(r"^\s+flat_(load|store|atomic)", m.group(2), re.M):
            out.append(m.group(1))
    return out


def test_checker_pins():
    desc = ("\t.amdhsa_kernel _Za\n\t\t.amdhsa_user_sgpr_dispatch_ptr 1\n\t\t.amdhsa_user_sgpr_queue_ptr 0\n"
            "\t.end_amdhsa_kernel\n\t.amdhsa_kernel _Zb\n\t\t.amdhsa_user_sgpr_dispatch_ptr 0\n"
            "\t.end_amdhsa_kernel\n")
    assert dispatch_ptr_kernels(desc) == ["_Za"]
    code = ("_Za:                  ; @_Za\n\tglobal_load_dword v1, v[2:3], off\n.Lfunc_end0:\n"
            "_Zb:                  ; @_Zb\n\tflat_load_dword v1, v[2:3]\n.Lfunc_end1:\n"
            "_Zc:\n\tds_read_b32 v1, v2\n\tflat_store_dword v[2:3], v1\n.Lfunc_end2:\n"
            "_Zf:\n\tflat_load_dword v1, v[2:3]\n.Lfunc_end3:\n"
            "\t.amdhsa_kernel _Za\n\t.end_amdhsa_kernel\n\t.amdhsa_kernel _Zb\n\t.end_amdhsa_kernel\n"
            "\t.amdhsa_kernel _Zc\n\t.end_amdhsa_kernel\n")
    assert flat_memory_kernels(code) == ["_Zb", "_Zc"]


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is not installed")
def test_no_dispatch_packet_reads_or_flat_memory(tmp_path):
    sys.path.insert(0, REPO)
    from kernelswift_amd import build as ksbuild
    srcs = sorted(glob.glob(os.path.join(REPO, "kernelswift_amd", "csrc", "*.hip")))
    assert srcs

    def compile_one(src):
        out = tmp_path / (os.path.basename(src) + ".s")
        r = subprocess.run([ksbuild.HIPCC, *ksbuild.COMMON, "--cuda-device-only", "-S", src, "-o", str(out)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        asm = out.read_text()
        return src, dispatch_ptr_kernels(asm), flat_memory_kernels(asm)

    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as ex:
        results = list(ex.map(compile_one, srcs))
    bad = [f"{os.path.basename(src)}: {k} (dispatch pointer)" for src, ks, _ in results for k in ks]
    bad += [f"{os.path.basename(src)}: {k} (flat memory instruction)" for src, _, fl in results for k in fl]
    assert bad == [], "\n".join(bad)
