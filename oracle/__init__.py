"""CPU oracle for the MuonAdamW step -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's hot path
(``MuonAdamW package/triton_muon_adamw``) so that the HIP kernels can be
checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as a checker.
The product (``triton-muonadamw_amd/``) never imports it and has no CPU
fallback.

Modules
-------
bf16    round-to-nearest-even bfloat16 emulation on float32 arrays
adamw   triton_adam.py:53-59 (update) and :132-153 (step loop semantics)
muon    triton_muon.py:327-372 / torch/optim/_muon.py:31-84,285-318
        (momentum, Nesterov blend, Newton-Schulz, LR scale, update)

Every function is pinned by tests in ``tests/test_oracle_*.py`` against
closed forms, invariants and the torch.optim library routines the reference
delegates to (``PyTorchMuonAdamW``, optimizer.py:178-260), and by the golden
fixtures in ``tests/golden/``.
"""

from . import adamw, bf16, muon  # noqa: F401
