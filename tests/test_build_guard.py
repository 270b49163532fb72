"""The product build refuses kernels that use scratch memory (CPU only: hipcc
cross-compiles for gfx950 without a GPU)."""

import shutil

import pytest

from triton_muon_adamw import _build

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
