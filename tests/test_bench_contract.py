"""bench.py's host-side contract, on the CPU: the one-GPU guard, the kernel
names its roofline object uses, and that those names resolve in the committed
rocprofv3 traffic summary (a renamed kernel would silently report
``traffic: null``)."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize("gpus", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(gpus):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(gpus)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_kernel_labels_follow_the_template_arguments():
    # variant = 8 * tile + (k-blocked | k-major << 1 | lower << 2); tile 192 is the 128 x 192 update tile
    assert bench.kernel_label("ns_gemm_kernel:update", 8 * 256 + 1 + 4) == "ns_gemm_kernel<256, 2, true, false, true, 256>"
    assert bench.kernel_label("ns_gemm_kernel:gram", 8 * 256 + 1 + 2) == "ns_gemm_kernel<256, 0, true, true, false, 256>"
    assert bench.kernel_label("ns_gemm_kernel:apply", 8 * 192 + 1 + 4) == "ns_gemm_kernel<128, 3, true, false, true, 192>"
    assert bench.kernel_label("ns_gemm_kernel:poly", 8 * 128 + 1 + 4) == "ns_gemm_kernel<128, 1, true, false, true, 128>"
    assert bench.kernel_label("adamw_mt_kernel", 0) == "adamw_mt_kernel"


@pytest.mark.parametrize("mode, variant", [("update", 8 * 256 + 5), ("apply", 8 * 256 + 5), ("gram", 8 * 256 + 3),
                                           ("poly", 8 * 256 + 5)])
def test_llama8b_gemms_have_committed_traffic(mode, variant):
    b = bench.traffic_bytes(bench.kernel_label(f"ns_gemm_kernel:{mode}", variant))
    assert b is not None and b > 1e9


def test_adamw_traffic_is_its_algorithmic_bytes():
    # 28 B per element over the Llama-8B AdamW set (1,050,939,392 elements), within the counters' rounding
    b = bench.traffic_bytes("adamw_mt_kernel")
    assert b is not None and abs(b / (28 * 1_050_939_392) - 1) < 0.01
