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
same compile checks that no kernel contains a flat memory instruction.

The score kernels issue their key-block loads before a barrier that orders them ahead of every wave's q loads (a
CU serves its loads in issue order, so waves whose key-block share queued behind the other waves' q rows would
hold up the block's staging).  Whether the compiler keeps the loads there depends on how their values are used:
with the values feeding only LDS stores it sank them below the q loads, and the 64-head bound kernel went from 60
to 64 us at config 4.  The same compile checks that the loads precede the barrier.

Some kernels' speed rests on their register, scratch and LDS budgets, which a small source change can break
silently (a lambda shared between two epilogues made the bound score kernel's tile loop reload spilled registers
every iteration: config 4's score kernel went from 61 to 76 us).  The same compile checks those budgets."""
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


def kernel_resources(asm: str):
    """{kernel name: (VGPRs, scratch bytes per lane, LDS bytes)} from the kernel descriptors."""
    out = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", asm, re.S):
        field = lambda f: int(re.search(r"\.amdhsa_" + f + r"\s+(\d+)", m.group(2)).group(1))
        out[m.group(1)] = (field("next_free_vgpr"), field("private_segment_fixed_size"),
                           field("group_segment_fixed_size"))
    return out


# (mangled-name fragment, what the budget buys, max VGPRs, max scratch bytes, max LDS bytes)
BUDGETS = [
    # bound score kernel, non-counting (config 4): three waves per SIMD; 8 bytes of scratch outside the tile loop
    ("indexer_scores_kernelILi4ELi128ELb0ELb1ELb0ELb0E", "3 waves/SIMD, no spill in the tile loop", 168, 8, 80 * 1024),
    # bound score kernel, counting (config 2): one workgroup per CU, no scratch
    ("indexer_scores_kernelILi4ELi128ELb0ELb1ELb1ELb0E", "no spill", 256, 0, 160 * 1024),
    # exact score kernel at the drop-in shape: four waves per SIMD, two workgroups per CU (scratch only on the
    # flush's rare wide-range paths)
    ("indexer_scores_kernelILi1ELi64ELb1ELb0ELb0ELb0E", "2 workgroups/CU at 4 waves/SIMD", 128, 32, 80 * 1024),
    # wave top-k: no scratch
    ("topk_wave_kernelILi12E", "no spill", 64, 0, 64 * 1024),
]


def test_checker_pins_resources():
    desc = ("\t.amdhsa_kernel _Za\n\t\t.amdhsa_group_segment_fixed_size 4096\n"
            "\t\t.amdhsa_private_segment_fixed_size 8\n\t\t.amdhsa_next_free_vgpr 97\n\t.end_amdhsa_kernel\n")
    assert kernel_resources(desc) == {"_Za": (97, 8, 4096)}


@pytest.fixture(scope="module")
def compiled(tmp_path_factory):
    """Every library source compiled for gfx950 with the library's flags: {source: assembly}."""
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc is not installed")
    sys.path.insert(0, REPO)
    from kernelswift_amd import build as ksbuild
    srcs = sorted(glob.glob(os.path.join(REPO, "kernelswift_amd", "csrc", "*.hip")))
    assert srcs
    tmp = tmp_path_factory.mktemp("asm")

    def compile_one(src):
        out = tmp / (os.path.basename(src) + ".s")
        r = subprocess.run([ksbuild.HIPCC, *ksbuild.flags(src), "--cuda-device-only", "-S", src, "-o", str(out)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return src, out.read_text()

    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as ex:
        return dict(ex.map(compile_one, srcs))


def test_no_dispatch_packet_reads_or_flat_memory(compiled):
    bad = [f"{os.path.basename(src)}: {k} (dispatch pointer)" for src, asm in compiled.items()
           for k in dispatch_ptr_kernels(asm)]
    bad += [f"{os.path.basename(src)}: {k} (flat memory instruction)" for src, asm in compiled.items()
            for k in flat_memory_kernels(asm)]
    assert bad == [], "\n".join(bad)


def loads_before_first_barrier(asm: str):
    """{kernel name: 16-byte global loads ahead of the kernel's first s_barrier}."""
    out = {}
    for m in re.finditer(r"^(\w+):[^\n]*\n(.*?)^\.Lfunc_end", asm, re.S | re.M):
        body = m.group(2)
        cut = re.search(r"^\s+s_barrier\b", body, re.M)
        if cut is not None:
            out[m.group(1)] = len(re.findall(r"^\s+global_load_dwordx4\b", body[:cut.start()], re.M))
    return out


def test_checker_pins_load_order():
    code = ("_Za:\n\tglobal_load_dwordx4 v[0:3], v[4:5], off\n\tglobal_load_dword v6, v[4:5], off\n\ts_barrier\n"
            "\tglobal_load_dwordx4 v[0:3], v[4:5], off\n.Lfunc_end0:\n"
            "_Zb:\n\ts_barrier\n\tglobal_load_dwordx4 v[0:3], v[4:5], off\n.Lfunc_end1:\n")
    assert loads_before_first_barrier(code) == {"_Za": 1, "_Zb": 0}


# (mangled-name fragment, 16-byte key-block loads per thread that must precede the first barrier)
LOAD_ORDER = [
    ("indexer_scores_kernelILi4ELi128ELb0ELb1ELb0ELb0E", 8),  # bound, config 4
    ("indexer_scores_kernelILi4ELi128ELb0ELb1ELb1ELb0E", 8),  # bound and counting, config 2
    ("indexer_scores_kernelILi4ELi128ELb0ELb0ELb0ELb0E", 8),  # exact, 64 heads
    ("indexer_scores_kernelILi1ELi64ELb1ELb0ELb0ELb0E", 4),   # exact, the drop-in shape
]


def test_key_block_loads_precede_the_ordering_barrier(compiled):
    found = {}
    for asm in compiled.values():
        found.update(loads_before_first_barrier(asm))
    bad = []
    for frag, n in LOAD_ORDER:
        hits = [(k, v) for k, v in found.items() if frag in k]
        assert hits, f"no kernel matches {frag}"
        bad += [f"{k}: {v} key-block loads before the barrier, {n} expected" for k, v in hits if v < n]
    assert bad == [], "\n".join(bad)


def test_register_scratch_and_lds_budgets(compiled):
    res = {}
    for asm in compiled.values():
        res.update(kernel_resources(asm))
    bad = []
    for frag, why, vmax, smax, lmax in BUDGETS:
        hits = [(k, r) for k, r in res.items() if frag in k]
        assert hits, f"no kernel matches {frag}"
        for k, (v, sc, lds) in hits:
            if v > vmax or sc > smax or lds > lmax:
                bad.append(f"{frag} ({why}): {v} VGPRs (max {vmax}), {sc} B scratch (max {smax}), "
                           f"{lds} B LDS (max {lmax})")
    assert bad == [], "\n".join(bad)
