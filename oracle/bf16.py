"""bfloat16 <-> float32 conversions on raw bit patterns (numpy has no bf16).

A bf16 array is carried as ``uint16`` holding the upper half of an IEEE fp32.
``f32_to_bf16`` rounds to nearest, ties to even, and keeps NaNs NaN (it sets the
quiet bit so a payload that lives only in the dropped half cannot become Inf).
This is the rounding every bf16 output of the HIP library uses.

Pinned by tests/test_oracle_bf16.py: exhaustive round trip of all 65536 bf16
patterns, torch's own ``float32 -> bfloat16`` cast (RNE) on random and tie
inputs, and hand-picked ties/overflow/NaN cases.
"""
import numpy as np


def bf16_to_f32(h):
    """uint16 bf16 bit patterns -> float32 (exact)."""
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(f):
    """float32 -> uint16 bf16 bit patterns, round-to-nearest-even, NaN kept."""
    f = np.ascontiguousarray(np.asarray(f, dtype=np.float32))
    u = f.view(np.uint32)
    is_nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    rounded = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    quiet = ((u >> np.uint32(16)) | np.uint32(0x0040)).astype(np.uint16)
    return np.where(is_nan, quiet, rounded).astype(np.uint16)


def round_bf16(f):
    """float -> nearest bf16 value, returned as float32."""
    return bf16_to_f32(f32_to_bf16(np.asarray(f, dtype=np.float32)))
