"""Static check of MFMA data hazards in compiled gfx950 assembly (test infrastructure).

Kernels that issue MFMAs from inline assembly keep them out of the compiler's hazard tracking: the compiler
does not insert the wait states that the CDNA3/CDNA4 ISA requires around them, and a register copy it
places between such an MFMA and the code's own NOP fence reads a result that is not written yet.  This
module parses a kernel's assembly (hipcc --cuda-device-only -S) into basic blocks and checks, along every
control-flow path:

  * after an MFMA, no instruction reads or writes its destination registers within MFMA_READ_WS wait
    states, except a later MFMA that accumulates into exactly the same registers (srcC == dst, which the
    hardware interlocks);
  * before an MFMA, no instruction writes its source registers within MFMA_SRC_WS wait states.

Wait states: one per issued instruction, N + 1 for `s_nop N`.  The limits are the conservative ones for
the 8-pass bf16 MFMAs used here (results read by VALU / memory instructions: 18 wait states for 16-pass
XDL ops, fewer for 8-pass; VALU writes of MFMA sources: 2).
"""
import re
from typing import Dict, List, Set, Tuple

MFMA_READ_WS = 19
MFMA_SRC_WS = 2

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_LABEL = re.compile(r"^(\.LBB[\w]+|\w[\w.$]*):")
_NO_FALLTHROUGH = ("s_branch", "s_endpgm", "s_setpc_b64")
_LOADS = ("ds_read", "global_load", "buffer_load", "scratch_load", "flat_load")


def _regs(text: str) -> Set[Tuple[str, int]]:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            k, lo, hi = m.group(1), int(m.group(2)), int(m.group(3))
            out.update((k, i) for i in range(lo, hi + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


class Inst:
    def __init__(self, text: str):
        self.text = text
        parts = text.split(None, 1)
        self.op = parts[0]
        ops = parts[1] if len(parts) > 1 else ""
        self.operands = [o.strip() for o in ops.split(",")] if ops else []
        self.is_mfma = self.op.startswith("v_mfma")
        if self.op == "s_nop":
            self.ws = int(self.operands[0], 0) + 1
        else:
            self.ws = 1
        self.dst: Set[Tuple[str, int]] = set()
        self.src: Set[Tuple[str, int]] = set()
        self.src_c: Set[Tuple[str, int]] = set()
        if not self.operands or self.op.startswith("s_"):
            return
        writes_first = not (self.op.startswith(("global_store", "buffer_store", "ds_write", "flat_store",
                                               "scratch_store", "global_atomic", "buffer_atomic",
                                               "ds_add", "ds_max", "ds_min", "ds_or", "ds_and"))
                            or self.op.startswith("v_cmpx"))
        if self.op.startswith("v_cmp") and not self.op.startswith("v_cmpx"):
            # VOPC writes vcc / an SGPR pair: no vector destination
            writes_first = False
        if writes_first:
            self.dst = _regs(self.operands[0])
            for o in self.operands[1:]:
                self.src |= _regs(o)
        else:
            for o in self.operands:
                self.src |= _regs(o)
        if self.is_mfma and len(self.operands) >= 4:
            self.src_c = _regs(self.operands[3])


def parse_kernel(asm: str, symbol: str) -> Tuple[List[List[Inst]], Dict[int, List[int]]]:
    """Basic blocks of `symbol` (instructions) and their successor lists."""
    lines = asm.splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith(symbol + ":"))
    end = next(i for i in range(start + 1, len(lines)) if lines[i].startswith(".Lfunc_end"))
    blocks: List[List[Inst]] = [[]]
    labels: Dict[str, int] = {}
    targets: List[List[str]] = [[]]
    falls: List[bool] = [True]
    for raw in lines[start + 1:end]:
        line = raw.split(";")[0].rstrip()
        if not line.strip():
            continue
        m = _LABEL.match(line)
        if m:
            if blocks[-1] or targets[-1]:
                blocks.append([])
                targets.append([])
                falls.append(True)
            labels[m.group(1)] = len(blocks) - 1
            continue
        text = line.strip()
        if text.startswith("."):
            continue
        ins = Inst(text)
        blocks[-1].append(ins)
        if ins.op.startswith("s_cbranch") or ins.op == "s_branch":
            targets[-1].append(ins.operands[0])
            if ins.op == "s_branch":
                falls[-1] = False
            blocks.append([])
            targets.append([])
            falls.append(True)
        elif ins.op in _NO_FALLTHROUGH:
            falls[-1] = False
            blocks.append([])
            targets.append([])
            falls.append(True)
    succ: Dict[int, List[int]] = {}
    for b in range(len(blocks)):
        s = [labels[t] for t in targets[b] if t in labels]
        if falls[b] and b + 1 < len(blocks):
            s.append(b + 1)
        succ[b] = s
    return blocks, succ


def _preds(succ: Dict[int, List[int]]) -> Dict[int, List[int]]:
    p: Dict[int, List[int]] = {b: [] for b in succ}
    for b, ss in succ.items():
        for s in ss:
            p[s].append(b)
    return p


def check(asm: str, symbol: str) -> List[str]:
    """Hazard violations in kernel `symbol` (empty list: none)."""
    blocks, succ = parse_kernel(asm, symbol)
    preds = _preds(succ)
    bad: List[str] = []

    def forward(b: int, i: int, ws: int, d: Set[Tuple[str, int]], src: Inst, seen: Set[Tuple[int, int, int]]):
        while True:
            if ws >= MFMA_READ_WS:
                return
            if i >= len(blocks[b]):
                for s in succ[b]:
                    key = (s, 0, ws)
                    if key not in seen:
                        seen.add(key)
                        forward(s, 0, ws, d, src, seen)
                return
            ins = blocks[b][i]
            touched = (ins.src | ins.dst) & d
            if touched:
                chained = ins.is_mfma and ins.dst == src.dst and ins.src_c == src.dst and not ((ins.src - ins.src_c) & d)
                if not chained:
                    bad.append(f"{symbol}: '{ins.text}' uses the result of '{src.text}' after {ws} wait states")
                    return
                return  # the chained MFMA takes over the registers (it is checked on its own)
            ws += ins.ws
            i += 1

    def backward(b: int, i: int, ws: int, s: Set[Tuple[str, int]], dst_mfma: Inst, seen: Set[Tuple[int, int, int]]):
        while True:
            if ws >= MFMA_SRC_WS:
                return
            if i < 0:
                for p in preds[b]:
                    key = (p, len(blocks[p]) - 1, ws)
                    if key not in seen:
                        seen.add(key)
                        backward(p, len(blocks[p]) - 1, ws, s, dst_mfma, seen)
                return
            ins = blocks[b][i]
            # loads are ordered by s_waitcnt (the compiler's waitcnt pass sees inline-asm operands), not by
            # wait states: only ALU writes count here
            if not ins.is_mfma and not ins.op.startswith(_LOADS) and ins.dst & s:
                bad.append(f"{symbol}: '{dst_mfma.text}' reads '{ins.text}' after {ws} wait states")
                return
            ws += ins.ws
            i -= 1

    for b, blk in enumerate(blocks):
        for i, ins in enumerate(blk):
            if not ins.is_mfma:
                continue
            forward(b, i + 1, 0, ins.dst, ins, {(b, i + 1, 0)})
            backward(b, i - 1, 0, ins.src, ins, {(b, i - 1, 0)})
    return bad


def kernel_symbols(asm: str, contains: str) -> List[str]:
    """Kernel symbols (definitions) whose mangled name contains `contains`."""
    return sorted({l.split(":")[0] for l in asm.splitlines()
                   if l.startswith("_Z") and ":" in l and contains in l.split(":")[0]})
