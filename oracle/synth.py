"""Seeded synthetic layer states for the parity tests (test infra only).

Follows the reference offline recipe: ``compute_smooth_scale``
(``quant/svd.py:26-30``), ``svd_lowrank`` (``:33-86``), residual + group-wise
INT4 + packing + storage dtypes (``scripts/convert_simulated.py:184-208``).

Choices (recorded because the reference leaves them open):

* smoothing follows the literal formula ``s = sqrt(amax|X_:,j| / amax|W_:,j|)``;
  ``smooth_clamp=(0.25, 4.0)`` reproduces the reference clamp instead (with the
  N(0,1)-with-outliers inputs it clamps every channel to 4.0);
* ``s`` is stored in bf16 and the migration ``W * s`` uses that stored value;
* the residual subtracts the bf16-rounded factors ``f32(L1) @ f32(L2)`` that
  the runtime will actually use;
* the rank-r factors come from ``torch.svd_lowrank`` (seeded, oversample 8,
  4 power iterations) or an exact SVD when the matrix is small.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16, fp16
from .pack import pack_int4, quantize_symmetric_int4
from .sim import Adapter, LayerState


def make_activation(m: int, k: int, seed: int = 0, outlier_frac: float = 0.01,
                    outlier_scale: float = 20.0, outlier_seed: int = 2) -> np.ndarray:
    """bf16 [m, k] ~ N(0,1) with round(outlier_frac * k) channels scaled by outlier_scale."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    n_out = int(round(outlier_frac * k))
    if n_out:
        cols = np.random.default_rng(outlier_seed).permutation(k)[:n_out]
        x[:, cols] *= np.float32(outlier_scale)
    return bf16(x)


def smooth_scale(x_absmax: np.ndarray, w: np.ndarray, clamp: tuple[float, float] | None = None):
    """``quant/svd.py:26-30``; unclamped unless ``clamp`` is given. Returns bf16 values."""
    w_absmax = np.maximum(np.abs(w).max(axis=0), np.float32(1e-8))
    s = np.sqrt(np.maximum(x_absmax.astype(np.float32), np.float32(1e-8)) / w_absmax)
    if clamp is not None:
        s = np.clip(s, clamp[0], clamp[1])
    return bf16(s.astype(np.float32))


def lowrank(w: np.ndarray, rank: int, seed: int = 3, oversample: int = 8, niter: int = 4):
    """Rank-r factors ``L1 = U_r S_r`` [N, r], ``L2 = V_r^T`` [r, K] (``quant/svd.py:33-86``)."""
    import torch

    wt = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32))
    min_dim = min(wt.shape)
    rank = max(1, min(int(rank), min_dim))
    q = min(rank + oversample, min_dim)
    if min_dim <= max(q, 32):
        u, s, vh = torch.linalg.svd(wt, full_matrices=False)
        u, s, vh = u[:, :rank], s[:rank], vh[:rank]
    else:
        gen_state = torch.random.get_rng_state()
        torch.manual_seed(seed)
        u, s, v = torch.svd_lowrank(wt, q=q, niter=niter)
        torch.random.set_rng_state(gen_state)
        u, s, vh = u[:, :rank], s[:rank], v[:, :rank].T
    return (u * s[None, :]).numpy(), vh.contiguous().numpy()


def make_layer(n: int, k: int, x_sample: np.ndarray, *, rank: int = 32, group_size: int = 64,
               seed: int = 1, w_std: float = 0.02, bias: bool = False,
               smooth_clamp: tuple[float, float] | None = None, svd_seed: int = 3) -> LayerState:
    """Quantize a seeded N(0, w_std) fp32 weight [n, k] the way ``convert_simulated.py`` does."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(w_std)).astype(np.float32)
    s = smooth_scale(np.abs(x_sample).max(axis=0), w, smooth_clamp)
    migrated = (w * s[None, :]).astype(np.float32)
    l1, l2 = lowrank(migrated, rank, seed=svd_seed)
    l1, l2 = bf16(l1), bf16(l2)
    residual = (migrated - l1.astype(np.float32) @ l2.astype(np.float32)).astype(np.float32)
    q, scales = quantize_symmetric_int4(residual, group_size, dtype="f32")
    b = None
    if bias:
        b = bf16(np.random.default_rng(seed + 100).standard_normal(n).astype(np.float32) * 0.1)
    return LayerState(smooth=s, qweight=pack_int4(q), weight_scales=fp16(scales), l1=l1, l2=l2,
                      bias=b, group_size=group_size, shape=(n, k))


def make_adapter(n: int, k: int, rank: int = 64, std: float = 0.01, scale: float = 0.8,
                 network_alpha: float | None = None, seed: int = 4) -> Adapter:
    """LoRA rank ``rank`` with A, B ~ N(0, std) stored in bf16 (benchmark config 4)."""
    rng = np.random.default_rng(seed)
    down = bf16(rng.standard_normal((rank, k), dtype=np.float32) * np.float32(std))
    up = bf16(rng.standard_normal((n, rank), dtype=np.float32) * np.float32(std))
    return Adapter(down=down, up=up, scale=scale, network_alpha=network_alpha)
