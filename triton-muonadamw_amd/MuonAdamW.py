"""Source-tree import of the packaged optimizer (mirrors the reference's MuonAdamW.py:3-10)."""

from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW

__all__ = [
    "AdamConfig",
    "MuonAdamW",
    "MuonConfig",
    "PyTorchMuonAdamW",
]
