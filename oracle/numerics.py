"""bf16 rounding on numpy float32 arrays (test infrastructure; see oracle/__init__.py)."""

import numpy as np


def to_bf16(a):
    """Round float32 values to the nearest bf16 (ties to even); returns float32 holding bf16 values.

    NaN stays NaN; values past the largest bf16 round to +-Inf, as IEEE rounding does.
    """
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32).copy()
    out[np.isnan(a)] = np.nan
    return out


def bf16_bits(a):
    """uint16 storage of bf16-valued float32 data (no rounding: call to_bf16 first)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits):
    """float32 values of uint16 bf16 storage."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
