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

Model: along one path through the code, every LGKM operation (``ds_*``,
scalar memory loads, ``s_memtime``...) joins an ordered list of outstanding
operations when issued; ``s_waitcnt ... lgkmcnt(N)`` retires all but the N
youngest, or nothing for N > 0 while a scalar memory load (which completes
out of order) or more than 32 operations are outstanding (a loop that issues
without waiting: its list is then kept as a set, so the analysis ends).  The
kernel body (from its symbol to its ``.Lfunc_end`` label, so blocks placed
after ``s_endpgm`` are covered) is cut into basic blocks: ``s_branch`` goes to its label only, ``s_cbranch_*`` to its
label or the next instruction, ``s_endpgm`` nowhere.  The state at a block's
entry is the set of outstanding lists of every path that reaches it,
iterated to a fixed point, so loops and branches are followed whatever their
layout; an instruction is a hazard if it touches a pending register in any of
them.  Any other transfer of control (``s_setpc``, a branch to an unknown
label) or a state that does not settle is reported as a hazard too.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

_LABEL = re.compile(r"^([.\w$]+):")
_BRANCH = re.compile(r"^s_(cbranch_\w+|branch)\s+([.\w$]+)")
_RANGE = re.compile(r"\bv\[(\d+):(\d+)\]")
_SINGLE = re.compile(r"\bv(\d+)\b")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")
_READ = re.compile(r"ds_read\w*\s+(v\[\d+:\d+\]|v\d+)\s*,\s*(v\d+)")
_SMEM = re.compile(r"s_(load|buffer_load|memtime|memrealtime|dcache)")
_MAX_ORDERED = 32   # outstanding operations a path keeps in issue order
_MAX_STATES = 4096  # outstanding lists per block entry before the analysis gives up


def _vregs(text: str) -> frozenset[int]:
    out: set[int] = set()
    for m in _RANGE.finditer(text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in _SINGLE.finditer(text):
        out.add(int(m.group(1)))
    return frozenset(out)


@dataclass(frozen=True)
class _Op:
    line: int        # issue line (1-based)
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


class _Decoded:
    """What the analysis needs of one instruction, parsed once."""

    __slots__ = ("line", "text", "kind", "regs", "op", "wait")

    def __init__(self, inst: _Inst, hazards: list[str]):
        self.line, self.text = inst.line, inst.text
        self.kind, self.regs, self.op, self.wait = "other", frozenset(), None, None
        t = inst.text
        if inst.in_asm and t.startswith("ds_read"):
            m = _READ.match(t)
            if not m:
                hazards.append(f"line {inst.line}: unparsed untracked read: {t}")
                return
            dest = _vregs(m.group(1))
            self.kind, self.regs, self.op = "read", dest | _vregs(m.group(2)), _Op(inst.line, "asm", dest)
        elif t.startswith("s_waitcnt"):
            m = _LGKM.search(t)
            self.kind, self.wait = "wait", (int(m.group(1)) if m else None)
        else:
            self.regs = _vregs(t)
            if t.startswith("ds_") and not t.startswith("ds_nop"):
                self.op = _Op(inst.line, "lds", frozenset())
            elif _SMEM.match(t):
                self.op = _Op(inst.line, "smem", frozenset())


def _step(d: _Decoded, seq, hazards: list[str]):
    """Apply one instruction to one path's outstanding operations (a tuple in
    issue order, or a frozenset once more than _MAX_ORDERED are outstanding:
    then only lgkmcnt(0) retires any); record hazards."""
    if d.kind == "wait":
        if d.wait is None:
            return seq
        if d.wait == 0:
            return ()
        if isinstance(seq, frozenset) or any(op.kind == "smem" for op in seq):
            return seq
        return seq[-d.wait:] if len(seq) > d.wait else seq
    if d.regs:
        for op in seq:
            if op.kind == "asm":
                for r in sorted(d.regs & op.dest):
                    hazards.append(f"line {d.line}: v{r} of the read at line {op.line} is still in flight: {d.text}")
    if d.op is None:
        return seq
    if isinstance(seq, frozenset):
        return seq | {d.op}
    return seq + (d.op,) if len(seq) < _MAX_ORDERED else frozenset(seq) | {d.op}


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


def _check_kernel(insts: list[_Inst], labels: dict[str, int], hazards: list[str]) -> None:
    n = len(insts)
    if n == 0:
        return
    dec = [_Decoded(i, hazards) for i in insts]
    # Basic blocks: leaders at the entry, at labels and after every transfer.
    leaders = {0} | {i for i in labels.values() if i < n}
    for i, inst in enumerate(insts):
        if _BRANCH.match(inst.text) or inst.text.startswith(("s_endpgm", "s_setpc", "s_swappc")):
            if i + 1 < n:
                leaders.add(i + 1)
    starts = sorted(leaders)
    block_of = {s: b for b, s in enumerate(starts)}
    ends = starts[1:] + [n]
    succ: list[list[int]] = []
    for s, e in zip(starts, ends):
        last = insts[e - 1]
        m = _BRANCH.match(last.text)
        nxt = [block_of[e]] if e < n else []
        if m:
            if m.group(2) not in labels or labels[m.group(2)] >= n:
                hazards.append(f"line {last.line}: branch to an unknown label: {last.text}")
                succ.append([])
                continue
            tgt = [block_of[labels[m.group(2)]]]
            succ.append(tgt if m.group(1) == "branch" else tgt + nxt)
        elif last.text.startswith("s_endpgm"):
            succ.append([])
        elif last.text.startswith(("s_setpc", "s_swappc")):
            hazards.append(f"line {last.line}: indirect transfer of control: {last.text}")
            succ.append([])
        else:
            succ.append(nxt)
    # Fixed point over the sets of outstanding lists at the block entries.
    entry: list[set] = [set() for _ in starts]
    entry[0].add(())
    work, queued = [0], {0}
    while work:
        b = work.pop()
        queued.discard(b)
        seqs = entry[b]
        for i in range(starts[b], ends[b]):
            seqs = {_step(dec[i], q, hazards) for q in seqs}
        last = insts[ends[b] - 1]
        if last.text.startswith("s_endpgm") and any(op.kind == "asm" for q in seqs for op in q):
            hazards.append(f"line {last.line}: kernel ends with untracked reads in flight")
        for t in succ[b]:
            new = seqs - entry[t]
            if new:
                entry[t] |= new
                if len(entry[t]) > _MAX_STATES:
                    hazards.append(f"line {insts[starts[t]].line}: outstanding LDS operations do not settle")
                    return
                if t not in queued:
                    work.append(t)
                    queued.add(t)


def check(asm: str, name_filter=("ns_gemm_kernel",)) -> Report:
    """Scan every kernel whose mangled name contains ``name_filter`` (a
    string or a tuple of them)."""
    rep = Report()
    for name, insts, labels in _kernels(asm, name_filter):
        rep.untracked_reads += sum(1 for i in insts if i.in_asm and i.text.startswith("ds_read"))
        hazards: list[str] = []
        _check_kernel(insts, labels, hazards)
        rep.hazards += [f"{name}: {h}" for h in dict.fromkeys(hazards)]
    return rep
