"""The inline-assembly MFMA kernels compile to code without MFMA data hazards (CPU: hipcc cross-compiles).

The MLA sparse-attention kernel issues its MFMAs from inline assembly (kernelswift_amd/csrc/sparse_attn.hip),
so the compiler's hazard recognizer does not cover them: a register copy the allocator places between such
an MFMA and the kernel's NOP fence would read an unfinished accumulator.  This compiles the source with the
library's own flags and checks every MLA kernel instantiation with tests/asm_hazards.py; the checker itself
is pinned on small synthetic programs first."""
import os
import shutil
import subprocess
import sys

import pytest

sys.path.insert(0, os.path.dirname(__file__))
import asm_hazards  # noqa: E402

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _prog(body: str) -> str:
    return "_Zk:\n" + body + "\n.Lfunc_end0:\n"


def test_checker_flags_early_read_and_accepts_fenced_read():
    mfma = "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n"
    early = _prog(mfma + "\tv_mov_b32 v1, v2\n\tv_accvgpr_read_b32 v0, a2\n\ts_endpgm")
    assert len(asm_hazards.check(early, "_Zk")) == 1
    fenced = _prog(mfma + "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\tv_accvgpr_read_b32 v0, a2\n\ts_endpgm")
    assert asm_hazards.check(fenced, "_Zk") == []
    # an accumulation chain into the same registers is interlocked by the hardware
    chain = _prog(mfma + mfma + "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\tv_accvgpr_read_b32 v0, a0\n\ts_endpgm")
    assert asm_hazards.check(chain, "_Zk") == []
    # the same MFMA result used as srcA is not
    bad_src = _prog(mfma + "\tv_mfma_f32_16x16x32_bf16 a[4:7], a[0:3], v[8:11], a[4:7]\n\ts_endpgm")
    assert len(asm_hazards.check(bad_src, "_Zk")) == 1


def test_checker_follows_branches():
    # the read sits behind a taken branch (loop exit): still within the window on that path
    prog = _prog("\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n"
                 "\ts_cbranch_scc1 .LBB0_2\n"
                 "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
                 ".LBB0_2:\n"
                 "\tv_accvgpr_read_b32 v0, a1\n\ts_endpgm")
    assert len(asm_hazards.check(prog, "_Zk")) == 1
    # VALU write of an MFMA source right before it
    prog2 = _prog("\tv_mov_b32 v5, 0\n\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n\ts_endpgm")
    assert len(asm_hazards.check(prog2, "_Zk")) == 1
    prog3 = _prog("\tv_mov_b32 v5, 0\n\ts_nop 1\n\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n"
                  "\ts_endpgm")
    assert asm_hazards.check(prog3, "_Zk") == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is not installed")
def test_mla_kernels_have_no_mfma_hazards(tmp_path):
    sys.path.insert(0, REPO)
    from kernelswift_amd import build as ksbuild
    src = os.path.join(REPO, "kernelswift_amd", "csrc", "sparse_attn.hip")
    out = tmp_path / "sparse_attn.s"
    cmd = [ksbuild.HIPCC, *ksbuild.flags(src), "--cuda-device-only", "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    syms = asm_hazards.kernel_symbols(asm, "sparse_attn_mla_kernel")
    assert len(syms) >= 4, syms
    bad = [v for s in syms for v in asm_hazards.check(asm, s)]
    assert bad == [], "\n".join(bad[:10])


def _m0_misuse(asm: str, symbol: str):
    """Instructions of `symbol` that touch m0 other than the LDS-DMA helper's own sequence
    (s_mov_b32 m0, ...; s_nop 0; global_load_lds_dwordx4): the helper declares m0 clobbered, which the
    compiler does not honour for a reserved register, so no compiler-generated use of m0 may exist."""
    blocks, _ = asm_hazards.parse_kernel(asm, symbol)
    bad = []
    for blk in blocks:
        for i, ins in enumerate(blk):
            if "m0" not in ins.operands:
                continue
            ok = (ins.op == "s_mov_b32" and ins.operands[0] == "m0" and i + 2 < len(blk)
                  and blk[i + 1].op == "s_nop" and blk[i + 2].op == "global_load_lds_dwordx4")
            if not ok:
                bad.append(f"{symbol}: '{ins.text}'")
    return bad


def test_m0_checker_pins():
    good = _prog("\ts_mov_b32 m0, s4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n\ts_endpgm")
    assert _m0_misuse(good, "_Zk") == []
    bad = _prog("\ts_mov_b32 m0, s4\n\tv_movrels_b32 v0, v1\n\ts_endpgm")
    assert len(_m0_misuse(bad, "_Zk")) == 1


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is not installed")
def test_lds_dma_kernels_use_m0_only_for_the_dma(tmp_path):
    sys.path.insert(0, REPO)
    from kernelswift_amd import build as ksbuild
    src = os.path.join(REPO, "kernelswift_amd", "csrc", "sparse_attn.hip")
    out = tmp_path / "sparse_attn_m0.s"
    r = subprocess.run([ksbuild.HIPCC, *ksbuild.flags(src), "--cuda-device-only", "-S", src, "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    syms = asm_hazards.kernel_symbols(asm, "sparse_attn")
    assert syms
    bad = [v for s in syms for v in _m0_misuse(asm, s)]
    assert bad == [], "\n".join(bad[:10])
