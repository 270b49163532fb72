"""MuonAdamW for AMD Instinct MI355X (gfx950), backed by hand-written HIP kernels.

Drop-in for the reference package ``triton_muon_adamw``
(``MuonAdamW package/triton_muon_adamw/__init__.py:3-9``): same exports, same
constructor, routing and step semantics.  The kernels live in
``libmuonadamw_amd.so`` (C ABI: ``include/muonadamw_amd.h``).
"""

from .optimizer import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW, split_parameters

__all__ = [
    "AdamConfig",
    "MuonAdamW",
    "MuonConfig",
    "PyTorchMuonAdamW",
    "split_parameters",
]
