"""bfloat16 emulation on float32 arrays (test infrastructure only).

bf16 keeps the top 16 bits of an IEEE float32.  ``round_bf16`` rounds to the
nearest representable value, ties to even -- the conversion torch uses for
``tensor.bfloat16()`` and the gfx950 ``v_cvt_pk_bf16_f32`` instruction
performs.  Values are returned as float32 arrays holding bf16-representable
numbers; ``to_bits`` / ``from_bits`` convert to and from the 16-bit patterns.
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """Round float32 values to bfloat16 (RNE); NaN stays NaN, inf stays inf."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32("nan")
    return out.reshape(np.shape(x))


def to_bits(x) -> np.ndarray:
    """bf16-representable float32 values -> uint16 bit patterns (exact)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bits(h) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)
