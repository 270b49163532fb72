"""The product build refuses kernels that use scratch memory, and GEMM
kernels whose untracked (inline-assembly) LDS reads have their registers used
before a wait that retires them (CPU only: hipcc cross-compiles for gfx950
without a GPU)."""

import shutil

import pytest

from triton_muon_adamw import _asmcheck, _build

SPILLING = r"""
#include <hip/hip_runtime.h>
// A private array indexed by a run-time value lives in scratch memory.
__global__ void spill_probe_kernel(float* out, int k) {
    float a[512];
    for (int i = 0; i < 512; ++i) a[i] = out[i * 7 + threadIdx.x];
    out[threadIdx.x] = a[(k + threadIdx.x) & 511];
}
"""

CLEAN = r"""
#include <hip/hip_runtime.h>
__global__ void clean_probe_kernel(float* out, float s) { out[threadIdx.x] *= s; }
"""

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not _build.Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc is not installed")


def test_remark_parser():
    remarks = ("a.hip:1:1: remark: Function Name: k1 [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:9:1: remark: Function Name: k2 [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 2064 [-Rpass-analysis=kernel-resource-usage]\n")
    assert _build.scratch_offenders(remarks) == [("k2", 2064)]


def test_build_rejects_a_spilling_kernel(tmp_path):
    src = tmp_path / "spill.hip"
    src.write_text(SPILLING)
    obj = tmp_path / "spill.o"
    with pytest.raises(RuntimeError, match="scratch memory.*spill_probe_kernel"):
        _build._compile(src, obj, verbose=False)
    assert not obj.exists()


def test_build_accepts_a_kernel_without_scratch(tmp_path):
    src = tmp_path / "clean.hip"
    src.write_text(CLEAN)
    obj = tmp_path / "clean.o"
    _build._compile(src, obj, verbose=False)
    assert obj.exists()


# ---- untracked LDS reads (inline assembly the compiler's wait-count pass does not see)

def _asm(body):
    return "_Zprobe_ns_gemm_kernel:\n" + body + "\ts_endpgm\n"


READ = ";;#ASMSTART\n\tds_read_b64_tr_b16 v[{0}:{1}], v5\n;;#ASMEND\n"


def test_checker_flags_a_use_before_the_wait():
    rep = _asmcheck.check(_asm(READ.format(10, 11) + "\tv_mov_b32 v20, v10\n\ts_waitcnt lgkmcnt(0)\n"))
    assert rep.untracked_reads == 1 and len(rep.hazards) == 1 and "v10" in rep.hazards[0]


def test_checker_retires_in_issue_order():
    # lgkmcnt(1) retires the older read only: its register is free, the younger one's is not.
    body = READ.format(10, 11) + READ.format(12, 13) + "\ts_waitcnt lgkmcnt(1)\n\tv_mov_b32 v20, v10\n"
    assert _asmcheck.check(_asm(body + "\ts_waitcnt lgkmcnt(0)\n")).hazards == []
    rep = _asmcheck.check(_asm(body + "\tv_mov_b32 v21, v12\n\ts_waitcnt lgkmcnt(0)\n"))
    assert len(rep.hazards) == 1 and "v12" in rep.hazards[0]


def test_checker_is_conservative_with_scalar_loads_and_branches():
    # A scalar load completes out of order: lgkmcnt(1) proves nothing about the read.
    body = READ.format(10, 11) + "\ts_load_dword s4, s[0:1], 0x0\n\ts_waitcnt lgkmcnt(1)\n\tv_mov_b32 v20, v10\n"
    assert len(_asmcheck.check(_asm(body + "\ts_waitcnt lgkmcnt(0)\n")).hazards) == 1
    # A loop whose next iteration reads the registers before any wait.
    loop = (".LBB0_1:\n\tv_mfma_f32_32x32x16_bf16 a[0:15], v[10:13], v[14:17], a[0:15]\n" + READ.format(10, 11)
            + "\ts_cbranch_scc1 .LBB0_1\n\ts_waitcnt lgkmcnt(0)\n")
    assert any("v10" in h for h in _asmcheck.check(_asm(loop)).hazards)
    # A forward branch that skips the wait carries its state to the target.
    fwd = (READ.format(10, 11) + "\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n.LBB0_2:\n"
           "\tv_mov_b32 v20, v10\n\ts_waitcnt lgkmcnt(0)\n")
    assert len(_asmcheck.check(_asm(fwd)).hazards) == 1


def test_checker_follows_unconditional_branches():
    # The block after an unconditional branch is reached only through its label: a use there is
    # judged with the state of the branches that reach it, not the state before the branch.
    skip = (READ.format(10, 11) + "\ts_branch .LBB0_3\n.LBB0_2:\n\tv_mov_b32 v10, 0\n\ts_endpgm\n"
            ".LBB0_3:\n\ts_waitcnt lgkmcnt(0)\n\ts_cbranch_scc1 .LBB0_2\n")
    assert _asmcheck.check(_asm(skip)).hazards == []
    # ... and a block placed after s_endpgm that a branch reaches before the wait is still checked.
    late = (READ.format(10, 11) + "\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n\ts_endpgm\n"
            ".LBB0_2:\n\tv_mov_b32 v20, v11\n\ts_waitcnt lgkmcnt(0)\n")
    rep = _asmcheck.check(_asm(late))
    assert len(rep.hazards) == 1 and "v11" in rep.hazards[0]


def test_checker_follows_every_path_around_a_loop():
    # The back edge reaches the use through a branch that skips the wait.
    loop = (".LBB0_1:\n\ts_cbranch_scc1 .LBB0_2\n\ts_waitcnt lgkmcnt(0)\n.LBB0_2:\n\tv_mov_b32 v20, v10\n"
            + READ.format(10, 11) + "\ts_cbranch_scc0 .LBB0_1\n\ts_waitcnt lgkmcnt(0)\n")
    rep = _asmcheck.check(_asm(loop))
    assert any("v10" in h and "v_mov_b32 v20, v10" in h for h in rep.hazards), rep.hazards
    # With the wait on both paths the same loop is clean.
    safe = loop.replace("\ts_cbranch_scc1 .LBB0_2\n", "")
    assert _asmcheck.check(_asm(safe)).hazards == []
    # A loop that issues reads into fresh registers and never waits inside
    # settles (its outstanding list becomes a set) and is caught at the end.
    grow = ".LBB0_1:\n" + READ.format(10, 11) + "\ts_cbranch_scc0 .LBB0_1\n"
    rep = _asmcheck.check(_asm(grow))
    assert any("ends with untracked reads in flight" in h for h in rep.hazards), rep.hazards


def test_checker_rejects_unknown_control_flow():
    rep = _asmcheck.check(_asm("\ts_cbranch_scc1 .LBB9_9\n"))
    assert any("unknown label" in h for h in rep.hazards)
    rep = _asmcheck.check(_asm("\ts_setpc_b64 s[0:1]\n"))
    assert any("indirect transfer" in h for h in rep.hazards)


PROBE = r"""
#include <hip/hip_runtime.h>
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2_t lds_read_tr16_untracked(unsigned a) {
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(a));
    return v;
}
__global__ void ns_gemm_kernel_probe(unsigned* out) {
    __shared__ unsigned short s[4096];
    s[threadIdx.x] = threadIdx.x;
    __syncthreads();
    u32x2_t v = lds_read_tr16_untracked(
        (unsigned)(size_t)(__attribute__((address_space(3))) void*)(s + (threadIdx.x & 63) * 4));
    WAIT
    out[threadIdx.x] = v.x + v.y;
}
"""


@pytest.mark.parametrize("wait,ok", [("", False), ("__builtin_amdgcn_s_waitcnt(0xC07F);", True)])
def test_build_check_on_compiled_code(tmp_path, wait, ok):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE.replace("WAIT", wait))
    if ok:
        _build._check_untracked_reads(src, verbose=False, out_dir=tmp_path)
    else:
        with pytest.raises(RuntimeError, match="untracked LDS reads used before their wait"):
            _build._check_untracked_reads(src, verbose=False, out_dir=tmp_path)
