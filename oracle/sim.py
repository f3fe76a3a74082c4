"""Restatement of the reference ``pytorch_sim`` forward and exact evaluators (test infra only).

* ``sim_forward_torch``: ``svdquant_linear_sim`` (``src/krea2_svdquant/quant/svd.py:119-163``)
  on CPU torch in the activation dtype, rounding where the reference rounds:
  ``x_hat = x / s`` (bf16), the residual weight dequantized in bf16
  (``pack.py:26-44`` with ``dtype=x.dtype``), three ``F.linear`` calls and a
  bf16 bias add.  The LoRA side branch follows ``runtime/linear.py:42-45`` and
  ``:156-161``: ``y + F.linear(F.linear(x, down), up) * mult`` on the *raw* x.
  This is the CPU path that ``bench.py`` times as its ``cpu_baseline``.
* ``w4a4_eval`` / ``w4a16_eval``: float64 evaluation of the quantized math
  (bf16 ``x_hat``, bit-exact A4 codes and bf16 scales for W4A4, the sim's bf16
  dequantized weight for W4A16), accumulation and the low-rank / LoRA
  branches in float64.  These are the references the GPU outputs are held to
  within a relative L2 error of 1e-3.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .numerics import bf16, from_bf16_bits, bf16_bits
from .pack import (dequantize_symmetric_int4, quantize_activations_a4, smooth_activations,
                   unpack_int4)


@dataclass
class Adapter:
    """LoRA side branch, ``runtime/linear.py:11-45`` (down [rl, K], up [N, rl])."""
    down: np.ndarray
    up: np.ndarray
    scale: float = 1.0
    network_alpha: float | None = None

    @property
    def rank(self) -> int:
        return int(self.down.shape[0])

    @property
    def multiplier(self) -> float:
        """``linear.py:38-40``: scale * alpha / rank, alpha defaulting to rank (``:34``)."""
        alpha = float(self.rank) if self.network_alpha is None else float(self.network_alpha)
        return float(self.scale) * (alpha / self.rank)


@dataclass
class LayerState:
    """Fields of ``SVDQuantLinearState`` (``quant/svd.py:12-23``) for a packed checkpoint layer.

    smooth bf16 [K]; qweight uint8 [N, Kp/2]; weight_scales fp16 [N, Kp/G];
    l1 bf16 [N, r]; l2 bf16 [r, K]; bias bf16 [N] or None.  Float arrays hold
    values exactly representable in the stored dtype.
    """
    smooth: np.ndarray
    qweight: np.ndarray
    weight_scales: np.ndarray
    l1: np.ndarray
    l2: np.ndarray
    bias: np.ndarray | None
    group_size: int
    shape: tuple[int, int]
    adapters: list[Adapter] = field(default_factory=list)

    @property
    def padded_in(self) -> int:
        """``runtime/load.py:111``: padded K = 2 * packed bytes per row."""
        return int(self.qweight.shape[1]) * 2

    def weight_codes(self) -> np.ndarray:
        return unpack_int4(self.qweight, self.padded_in)


def _pad_k(a: np.ndarray, kp: int) -> np.ndarray:
    if a.shape[-1] == kp:
        return a
    return np.concatenate([a, np.zeros(a.shape[:-1] + (kp - a.shape[-1],), a.dtype)], axis=-1)


def quantize_activations(x: np.ndarray, st: LayerState):
    """Smoothing + A4 quantization of a [M, K] bf16 activation.

    Returns ``(x_hat, packed [M, Kp/2], scales [M, Kp/G], codes [M, Kp])``.
    """
    x_hat = smooth_activations(x, st.smooth)
    packed, scales, codes = quantize_activations_a4(_pad_k(x_hat, st.padded_in), st.group_size)
    return x_hat, packed, scales, codes


def _lowrank_and_lora_f64(x: np.ndarray, x_hat: np.ndarray, st: LayerState):
    mid = x_hat.astype(np.float64) @ st.l2.astype(np.float64).T
    y = mid @ st.l1.astype(np.float64).T
    if st.bias is not None:
        y = y + st.bias.astype(np.float64)[None, :]
    for ad in st.adapters:
        down = bf16(ad.down).astype(np.float64)   # linear.py:43-44 casts to x.dtype
        up = bf16(ad.up).astype(np.float64)
        y = y + ad.multiplier * ((x.astype(np.float64) @ down.T) @ up.T)
    return y, mid


def w4a4_eval(x: np.ndarray, st: LayerState) -> dict:
    """Float64 value of the W4A4 layer on bf16 input ``x`` [M, K].

    ``y = sum_g sx[m,g] sw[n,g] sum_{k in g} qx[m,k] qw[n,k] + (x_hat L2^T) L1^T + bias
    + sum_a mult_a (x A_a^T) B_a^T``.  Every product sx*sw*qx*qw is exact in float64,
    so the group-wise sum equals one float64 GEMM of the scaled codes.
    """
    n, k = st.shape
    x_hat, packed, sx, qx = quantize_activations(x, st)
    g = st.group_size
    a = (qx.astype(np.float64).reshape(qx.shape[0], -1, g) * sx.astype(np.float64)[..., None])
    qw = st.weight_codes()
    b = (qw.astype(np.float64).reshape(n, -1, g) * st.weight_scales.astype(np.float64)[..., None])
    y_res = a.reshape(qx.shape[0], -1) @ b.reshape(n, -1).T
    y_lr, mid = _lowrank_and_lora_f64(x, x_hat, st)
    return {"y": y_res + y_lr, "y_res": y_res, "mid": mid, "x_hat": x_hat,
            "qx_packed": packed, "sx": sx, "qx": qx}


def sim_weight(st: LayerState) -> np.ndarray:
    """The sim's dequantized residual weight in bf16 (``svd.py:129-135``), [N, K]."""
    w = dequantize_symmetric_int4(st.weight_codes(), st.weight_scales, st.group_size, dtype="bf16")
    return w[:, : st.shape[1]]


def w4a16_eval(x: np.ndarray, st: LayerState) -> dict:
    """Float64 value of the W4A16 layer: the sim's bf16 operands, float64 accumulation."""
    x_hat = smooth_activations(x, st.smooth)
    y_res = x_hat.astype(np.float64) @ sim_weight(st).astype(np.float64).T
    y_lr, mid = _lowrank_and_lora_f64(x, x_hat, st)
    return {"y": y_res + y_lr, "y_res": y_res, "mid": mid, "x_hat": x_hat}


def sim_forward_torch(x, st: LayerState, *, num_threads: int | None = None):
    """``svdquant_linear_sim`` + LoRA adapters on CPU torch, in x's dtype.

    ``x`` is a torch tensor (bf16 in every configuration used here).  The steps
    and their roundings follow ``quant/svd.py:121-133,158-163`` and
    ``runtime/linear.py:42-45,158-160``.
    """
    import torch
    import torch.nn.functional as F

    if num_threads is not None:
        torch.set_num_threads(num_threads)
    dt = x.dtype

    def t(a, dtype=dt):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype)

    x_hat = x / t(st.smooth)
    q = torch.from_numpy(st.weight_codes())
    n, kp = q.shape
    g = st.group_size
    w = (q.reshape(n, kp // g, g).to(dt) * t(st.weight_scales, torch.float16).to(dt).unsqueeze(-1))
    w = w.reshape(n, kp)[:, : st.shape[1]]
    y = F.linear(x_hat, w) + F.linear(F.linear(x_hat, t(st.l2)), t(st.l1))
    if st.bias is not None:
        y = y + t(st.bias)
    for ad in st.adapters:
        y = y + F.linear(F.linear(x, t(ad.down)), t(ad.up)) * ad.multiplier
    return y


def quantize_activations_torch(x, st: LayerState, *, num_threads: int | None = None):
    """The A4 step on CPU torch, with the reference's own ops: ``x / smooth`` in x's dtype
    (``quant/svd.py:121-122``), then ``quantize_symmetric_int4(x_hat, G)`` (``quant/pack.py:6-23``:
    group ``amax``, ``clamp_min(1e-8) / 7`` in the input dtype, ``round(x_hat.float() / scales)``,
    clamp to [-8, 7]) and ``pack_int4`` (``pack.py:47-56``).  ``x`` is a bf16 torch tensor
    [M, K]; returns ``(packed uint8 [M, Kp/2], scales bf16 [M, Kp/G])`` as torch tensors.  The
    multithreaded CPU baseline of the activation pass; bit-identical to ``quantize_activations``.
    """
    import torch

    if num_threads is not None:
        torch.set_num_threads(num_threads)
    smooth = torch.from_numpy(np.ascontiguousarray(st.smooth, dtype=np.float32)).to(x.dtype)
    x_hat = x / smooth
    kp, g = st.padded_in, st.group_size
    if x_hat.shape[-1] != kp:
        x_hat = torch.cat([x_hat, x_hat.new_zeros(x_hat.shape[0], kp - x_hat.shape[-1])], dim=-1)
    grouped = x_hat.reshape(x_hat.shape[0], kp // g, g)
    scales = grouped.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 7.0
    q = torch.round(grouped.float() / scales).clamp(-8, 7).to(torch.int8).reshape(x_hat.shape[0], kp)
    u = (q.to(torch.int16) + 8).to(torch.uint8)
    packed = u[:, 0::2] | (u[:, 1::2] << 4)
    return packed, scales.squeeze(-1)


def rel_l2(a, b) -> float:
    """||a - b||_2 / ||b||_2 in float64."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


__all__ = ["Adapter", "LayerState", "quantize_activations", "quantize_activations_torch", "w4a4_eval", "w4a16_eval",
           "sim_weight", "sim_forward_torch", "rel_l2", "bf16_bits", "from_bf16_bits"]
