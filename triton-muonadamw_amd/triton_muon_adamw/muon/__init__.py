"""Muon branch (gfx950 HIP momentum + Newton-Schulz MFMA kernels)."""

from .hip_muon import (
    HipMuon,
    TritonMuon,
    muon_step,
    newton_shultz_step,
    solve_ns_kernel_1,
    solve_ns_kernel_2,
    solve_ns_kernel_3,
)

__all__ = [
    "HipMuon",
    "TritonMuon",
    "muon_step",
    "newton_shultz_step",
    "solve_ns_kernel_1",
    "solve_ns_kernel_2",
    "solve_ns_kernel_3",
]
