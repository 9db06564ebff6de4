"""Round-to-nearest-even bfloat16 and float16 emulation on float32 arrays (oracle infrastructure).

The reference's cast points (`.astype(compute)`, with the compute role bf16, fp16 or fp32 in its presets,
sa3jax/dtypes.py:23-58) are modelled by `round_bf16` and `round_fp16`, which return float32 arrays whose values
are exactly representable in the narrower type.
"""
from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float -> nearest bfloat16 (ties to even), returned as float32. NaN stays NaN, inf stays inf."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = rounded.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.nan
    return out


def round_fp16(x: np.ndarray) -> np.ndarray:
    """float -> nearest IEEE half (ties to even; overflow to inf, gradual underflow), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


COMPUTE = ("bf16", "fp16", "fp32")


def cast(x: np.ndarray, compute: str) -> np.ndarray:
    """Cast to the compute dtype ('bf16', 'fp16' or 'fp32'), returned as float32."""
    if compute == "bf16":
        return round_bf16(x)
    if compute == "fp16":
        return round_fp16(x)
    if compute == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"compute must be one of {COMPUTE}, got {compute!r}")


def to_bits(x: np.ndarray) -> np.ndarray:
    """bf16-representable float32 -> uint16 bit patterns (the upper half of each float32)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32."""
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)
