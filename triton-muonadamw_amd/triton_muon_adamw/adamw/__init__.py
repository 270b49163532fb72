"""AdamW branch (gfx950 HIP multi-tensor kernel)."""

from .hip_adam import HipAdamW, TritonAdamW, solve_adamw_step

__all__ = ["HipAdamW", "TritonAdamW", "solve_adamw_step"]
