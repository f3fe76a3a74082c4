"""Restatement of the reference INT4 quantizer and nibble packing (test infra only).

Follows ``src/krea2_svdquant/quant/pack.py`` of the reference:

* ``quantize_symmetric_int4``  -> ``pack.py:6-23``
* ``dequantize_symmetric_int4`` -> ``pack.py:26-44``
* ``pack_int4``                -> ``pack.py:47-56``
* ``unpack_int4``              -> ``pack.py:59-70``

plus ``quantize_activations_a4``: the same quantizer applied per group along K
to the smoothed bf16 activation ``x_hat`` (``quant/svd.py:121-122``), followed
by ``pack_int4`` -- the dynamic A4 step the reference plans in
``README.md:188-195`` but never implements.

Arrays are numpy.  The ``dtype`` argument names the torch dtype the reference
tensor would have ("bf16", "fp16" or "f32"); values are carried as float32
arrays holding values exactly representable in that dtype, and every
intermediate is rounded where torch rounds it:

* bf16/fp16 input: ``amax`` is exact, ``clamp_min(1e-8)`` yields
  ``max(amax, round(1e-8))``, the ``/ 7.0`` is an IEEE float32 division rounded
  once more to the input dtype, and the codes divide ``float32(x)`` by
  ``float32(scale)`` (IEEE), round half to even and clamp to [-8, 7];
* f32 input: the same in float32 with float32 scales.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16, fp16

_ROUND = {"bf16": bf16, "fp16": fp16, "f32": lambda a: np.asarray(a, dtype=np.float32)}


def _round_to(dtype: str):
    if dtype not in _ROUND:
        raise ValueError(f"unsupported dtype {dtype!r}")
    return _ROUND[dtype]


def pad_to_group(x: np.ndarray, group_size: int) -> np.ndarray:
    """Zero-pad the last dim to a multiple of ``group_size`` (``pack.py:12-16``)."""
    k = x.shape[-1]
    if k % group_size == 0:
        return x
    pad = group_size - k % group_size
    return np.concatenate([x, np.zeros(x.shape[:-1] + (pad,), dtype=x.dtype)], axis=-1)


def quantize_symmetric_int4(x: np.ndarray, group_size: int = 128, dtype: str = "f32"):
    """Group-wise symmetric INT4 along the last dim; returns (int8 codes, scales).

    ``pack.py:6-23``: ``scales = amax.clamp_min(1e-8) / 7``;
    ``q = round(x.float() / scales).clamp(-8, 7)``.
    Scales are returned as float32 values of ``dtype`` (bf16 for bf16 input).
    """
    rnd = _round_to(dtype)
    x = pad_to_group(np.asarray(x, dtype=np.float32), group_size)
    lead, k = x.shape[:-1], x.shape[-1]
    g = x.reshape(*lead, k // group_size, group_size)
    amax = np.abs(g).max(axis=-1)
    floor = float(rnd(np.float32(1e-8)))
    scales = rnd(np.maximum(amax, np.float32(floor)) / np.float32(7.0))
    q = np.rint(g / scales[..., None])
    q = np.clip(q, -8, 7).astype(np.int8).reshape(*lead, k)
    return q, scales.astype(np.float32)


def dequantize_symmetric_int4(q: np.ndarray, scales: np.ndarray, group_size: int = 128,
                              dtype: str = "f32") -> np.ndarray:
    """``pack.py:26-44``: ``q.to(dt) * scales.to(dt)``, the product rounded to ``dt``."""
    rnd = _round_to(dtype)
    lead, k = q.shape[:-1], q.shape[-1]
    g = rnd(q.astype(np.float32)).reshape(*lead, k // group_size, group_size)
    y = rnd(g * rnd(scales)[..., None])
    return y.reshape(*lead, k)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """``pack.py:47-56``: byte j = (q[2j]+8) | (q[2j+1]+8) << 4 (odd K zero-padded)."""
    q = np.asarray(q)
    if q.dtype != np.int8:
        raise TypeError("q must be int8")
    if q.shape[-1] % 2:
        q = np.concatenate([q, np.zeros(q.shape[:-1] + (1,), dtype=np.int8)], axis=-1)
    u = (q.astype(np.int16) + 8).astype(np.uint8)
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray, values_last_dim: int | None = None) -> np.ndarray:
    """``pack.py:59-70``: inverse of ``pack_int4`` (low nibble = even index)."""
    packed = np.asarray(packed)
    if packed.dtype != np.uint8:
        raise TypeError("packed must be uint8")
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = (packed & 0x0F).astype(np.int16) - 8
    out[..., 1::2] = ((packed >> 4) & 0x0F).astype(np.int16) - 8
    if values_last_dim is not None:
        out = out[..., :values_last_dim]
    return out


def smooth_activations(x: np.ndarray, smooth: np.ndarray) -> np.ndarray:
    """``quant/svd.py:121-122`` for bf16 x and bf16 s: ``bf16(float32(x) / float32(s))``."""
    return bf16(np.asarray(x, dtype=np.float32) / np.asarray(smooth, dtype=np.float32))


def quantize_activations_a4(x_hat: np.ndarray, group_size: int = 64):
    """Dynamic A4 step: per-group INT4 codes of bf16 ``x_hat`` along K, packed.

    Returns ``(packed uint8 [..., K/2], scales [..., K/G] as bf16 values, codes int8)``.
    """
    q, s = quantize_symmetric_int4(x_hat, group_size, dtype="bf16")
    return pack_int4(q), s, q
