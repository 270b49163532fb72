"""Build ``libmuonadamw_amd.so`` in-tree with hipcc for gfx950.

The library holds the HIP kernels and the C ABI declared in
``include/muonadamw_amd.h``.  It is built in place (next to this file) so the
same file is what tests, ``bench.py`` and the Python package load.

Usage: ``python -m triton_muon_adamw._build`` (with ``triton-muonadamw_amd`` on
``sys.path``) or ``build()`` from Python.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT_PKG = PKG_DIR.parent                      # triton-muonadamw_amd/
CSRC = ROOT_PKG / "csrc"
REPO = ROOT_PKG.parent
INCLUDE = REPO / "include"
BUILD_DIR = ROOT_PKG / "_build"
LIB_NAME = "libmuonadamw_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"

SOURCES = ["mamw_plan.cpp", "abi.cpp", "prof.cpp", "adamw.hip", "muon.hip"]

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
# Device code: gfx950 only; packed-fp32 instructions disabled (the compiler
# still emits ordinary scalar and vector fp32 code).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Per-kernel register / LDS / scratch report, read by scratch_offenders().
    "-Rpass-analysis=kernel-resource-usage",
]


def scratch_offenders(remarks: str) -> list[tuple[str, int]]:
    """Kernels whose resource-usage remark reports private scratch memory.

    Returns ``(mangled kernel name, bytes per lane)`` for every kernel with a
    non-zero ``ScratchSize``.  No kernel of this library may use scratch: a
    GEMM whose accumulators or fragments spill runs many times slower (a
    spilling variant of the Newton-Schulz GEMM once took minutes per launch),
    so a build that would produce one fails instead.
    """
    out: list[tuple[str, int]] = []
    name = None
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name is not None and int(m.group(1)) > 0:
            out.append((name, int(m.group(1))))
    return out


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MuonAdamW HIP library cannot be built")


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [_hipcc(), *COMMON_FLAGS]
    if src.suffix == ".hip":
        cmd += HIP_FLAGS + ["-x", "hip"]
    else:
        # Host-only C++: HIP runtime API headers, no device compilation.
        cmd += ["-x", "c++", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]
    cmd += ["-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    bad = scratch_offenders(res.stderr)
    if bad:
        obj.unlink(missing_ok=True)
        raise RuntimeError(f"{src.name}: kernels use scratch memory (spilled registers or private arrays), "
                           "which this library does not allow: "
                           + ", ".join(f"{n} ({b} bytes/lane)" for n, b in bad))
    if verbose and res.stderr.strip():
        # hipcc's host pass warns that it does not know the packed-fp32 feature;
        # the resource-usage remarks were checked above.
        lines = [ln for ln in res.stderr.splitlines()
                 if "packed-fp32-ops" not in ln and "kernel-resource-usage" not in ln]
        if any(ln.strip() for ln in lines):
            print("\n".join(lines), flush=True)


def _check_untracked_reads(src: Path, verbose: bool, out_dir: Path = BUILD_DIR) -> None:
    """Compile ``src``'s device code to assembly and verify its untracked LDS
    reads (inline assembly the compiler's wait-count pass does not see): no
    instruction may touch their registers before a wait that retires them."""
    from . import _asmcheck

    out = out_dir / (src.name + ".s")
    cmd = [_hipcc(), *COMMON_FLAGS, *HIP_FLAGS[:-1], "-x", "hip", "--cuda-device-only", "-S", str(src),
           "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    rep = _asmcheck.check(out.read_text())
    if rep.untracked_reads == 0:
        raise RuntimeError(f"{src.name}: no untracked LDS reads found in the GEMM kernels' assembly "
                           "(the check would be vacuous)")
    if rep.hazards:
        raise RuntimeError(f"{src.name}: registers of untracked LDS reads used before their wait:\n"
                           + "\n".join(rep.hazards[:20]))


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    jobs = min(len(SOURCES) + 1, max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for name in SOURCES:
            src = CSRC / name
            obj = BUILD_DIR / (name + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, src, obj, verbose))
            if "lds_read_tr16_untracked(" in src.read_text():
                futs.append(ex.submit(_check_untracked_reads, src, verbose))
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_name(LIB_NAME + ".tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
