"""bfloat16 bit patterns on numpy arrays (TEST INFRASTRUCTURE ONLY).

bf16 tensors are held as uint16 arrays of IEEE bfloat16 bit patterns.
Rounding is to nearest even, NaN -> 0x7fc0 (torch's c10::BFloat16 rule).
"""
from __future__ import annotations

import numpy as np


def to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def from_f32(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def round_f32(f: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 -> float32."""
    return to_f32(from_f32(f))


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in bf16 ulps, via the monotone integer order of the patterns."""
    def key(h):
        h = np.asarray(h, dtype=np.uint16).astype(np.int32)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + h)
    return np.abs(key(a) - key(b))
