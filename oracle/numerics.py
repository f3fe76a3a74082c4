"""Bit-exact bf16 / fp16 rounding in numpy (test infrastructure only).

bf16 values are carried as float32 arrays whose values are exactly
representable in bf16; ``bf16_bits`` / ``from_bf16_bits`` convert to and from
the uint16 storage form.  Rounding is IEEE round-to-nearest-even, which is what
torch uses for ``.to(torch.bfloat16)`` and for every bf16 arithmetic result on
the CPU (compute in float32, round once).
"""
from __future__ import annotations

import numpy as np


def bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 storage bits (uint16), round-to-nearest-even, NaN kept quiet."""
    f = np.asarray(a, dtype=np.float32)
    shape = f.shape
    f = np.ascontiguousarray(f).reshape(-1)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(f)
    out = rounded.astype(np.uint16)
    if nan.any():
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out.reshape(shape)


def from_bf16_bits(b) -> np.ndarray:
    """bf16 storage bits (uint16) -> float32 values (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32).reshape(b.shape)


def bf16(a) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (RNE); result is float32."""
    return from_bf16_bits(bf16_bits(a))


def fp16(a) -> np.ndarray:
    """Round float32 values to the nearest fp16 value (RNE); result is float32."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


BF16_1E_8 = float(bf16(np.float32(1e-8)))
"""``bf16(1e-8)``: the clamp floor a bf16 ``clamp_min(1e-8)`` produces."""
