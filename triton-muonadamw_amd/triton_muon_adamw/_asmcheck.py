"""Build-time check of the LDS reads that the compiler does not track.

Some LDS reads in the GEMM loop are issued as inline assembly
(``lds_read_tr16_untracked`` in ``csrc/muon.hip``) so that the compiler's
wait-count pass does not make them wait for the LDS DMA in flight.  The
compiler then also believes their destination registers are written at
issue, so nothing stops it from reading, copying or reusing those registers
before the data has arrived; the kernel source waits itself
(``s_waitcnt lgkmcnt``) before the MFMAs that consume them.  This module reads
the device assembly of the build and reports every instruction that touches
such a register while the read may still be in flight.

Model: every LGKM operation (``ds_*``, scalar memory loads, ``s_memtime``...)
joins an ordered list when issued; ``s_waitcnt ... lgkmcnt(N)`` retires all
but the N youngest, or nothing for N > 0 while a scalar memory load (which
completes out of order) is outstanding.  The scan follows the code in order;
at a forward branch the outstanding list is remembered and merged into the
state at its target label, and a backward branch re-scans from its target
with the branch's state until everything pending has been retired.  Nothing
falls through an unconditional branch or ``s_endpgm``: the block after one is
reached through its label only.  A kernel is scanned up to its
``.Lfunc_end`` label, so blocks placed after ``s_endpgm`` are covered.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

_LABEL = re.compile(r"^([.\w$]+):")
_BRANCH = re.compile(r"^s_(?:cbranch_\w+|branch)\s+([.\w$]+)")
_RANGE = re.compile(r"\bv\[(\d+):(\d+)\]")
_SINGLE = re.compile(r"\bv(\d+)\b")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def _vregs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _RANGE.finditer(text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in _SINGLE.finditer(text):
        out.add(int(m.group(1)))
    return out


@dataclass(frozen=True)
class _Op:
    line: int        # issue line (1-based), also the order of issue
    kind: str        # "asm" (untracked LDS read), "lds" or "smem"
    dest: frozenset  # destination VGPRs of an untracked read


@dataclass
class _Inst:
    line: int
    text: str
    in_asm: bool


@dataclass
class Report:
    untracked_reads: int = 0
    hazards: list[str] = field(default_factory=list)


def _retire(state: list[_Op], n: int) -> list[_Op]:
    if n == 0:
        return []
    if any(op.kind == "smem" for op in state):
        return state
    return state[-n:] if len(state) > n else state


def _merge(a: list[_Op], b: list[_Op]) -> list[_Op]:
    return sorted(set(a) | set(b), key=lambda op: op.line)


def _step(inst: _Inst, state: list[_Op], hazards: list[str]) -> list[_Op]:
    """Apply one instruction to the outstanding list; record hazards."""
    text = inst.text
    pending = {r: op.line for op in state if op.kind == "asm" for r in op.dest}
    if inst.in_asm and text.startswith("ds_read"):
        m = re.match(r"ds_read\w*\s+(v\[\d+:\d+\]|v\d+)\s*,\s*(v\d+)", text)
        if not m:
            hazards.append(f"line {inst.line}: unparsed untracked read: {text}")
            return state
        dest, addr = _vregs(m.group(1)), _vregs(m.group(2))
        for r in sorted((dest | addr) & set(pending)):
            hazards.append(f"line {inst.line}: v{r} of the read at line {pending[r]} is still in flight: {text}")
        return state + [_Op(inst.line, "asm", frozenset(dest))]
    if text.startswith("s_waitcnt"):
        m = _LGKM.search(text)
        return _retire(state, int(m.group(1))) if m else state
    touched = _vregs(text) & set(pending)
    for r in sorted(touched):
        hazards.append(f"line {inst.line}: v{r} of the read at line {pending[r]} is still in flight: {text}")
    if text.startswith("ds_") and not text.startswith("ds_nop"):
        return state + [_Op(inst.line, "lds", frozenset())]
    if re.match(r"s_(load|buffer_load|memtime|memrealtime|dcache)", text):
        return state + [_Op(inst.line, "smem", frozenset())]
    return state


def _kernels(asm: str, name_filter):
    """Yield (kernel name, instructions, label -> index) for each kernel body:
    everything from the kernel's symbol to its ``.Lfunc_end`` label, so the
    blocks the compiler places after ``s_endpgm`` (reached only by branches)
    are scanned too."""
    names = (name_filter,) if isinstance(name_filter, str) else tuple(name_filter)
    cur, insts, labels, in_asm = None, [], {}, False
    for no, raw in enumerate(asm.splitlines(), 1):
        line = raw.strip()
        m = _LABEL.match(raw)
        if m and raw[0] not in " \t" and m.group(1).startswith("_Z"):
            if cur is not None:
                yield cur, insts, labels
            cur = m.group(1) if any(n in m.group(1) for n in names) else None
            insts, labels, in_asm = [], {}, False
            continue
        if cur is None:
            continue
        if m and m.group(1).startswith(".Lfunc_end"):
            yield cur, insts, labels
            cur = None
            continue
        if line.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if line.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if m:
            labels[m.group(1)] = len(insts)
            continue
        code = line.split(";")[0].strip()
        if not code or code.startswith("."):
            continue
        insts.append(_Inst(no, code, in_asm))
    if cur is not None:
        yield cur, insts, labels


def check(asm: str, name_filter=("ns_gemm_kernel",)) -> Report:
    """Scan every kernel whose mangled name contains ``name_filter`` (a
    string or a tuple of them)."""
    rep = Report()
    for name, insts, labels in _kernels(asm, name_filter):
        hazards: list[str] = []
        state: list[_Op] = []
        at_label: dict[int, list[_Op]] = {}
        for i, inst in enumerate(insts):
            if i in at_label:
                state = _merge(state, at_label.pop(i))
            state = _step(inst, state, hazards)
            if inst.in_asm and inst.text.startswith("ds_read"):
                rep.untracked_reads += 1
            b = _BRANCH.match(inst.text)
            if b and b.group(1) in labels:
                t = labels[b.group(1)]
                if t > i:
                    at_label[t] = _merge(at_label.get(t, []), state)
                elif any(op.kind == "asm" for op in state):
                    # Back edge: the loop head runs again with this state.
                    s2 = list(state)
                    for j in range(t, i + 1):
                        s2 = _step(insts[j], s2, hazards)
                        if not any(op.kind == "asm" for op in s2):
                            break
            if inst.text.startswith("s_endpgm"):
                if any(op.kind == "asm" for op in state):
                    hazards.append(f"line {inst.line}: kernel ends with untracked reads in flight")
                state = []  # nothing falls through: the next block is reached by branches only
            elif b and inst.text.startswith("s_branch"):
                state = []  # unconditional: the next block is reached by branches only
        rep.hazards += [f"{name}: {h}" for h in dict.fromkeys(hazards)]
    return rep
