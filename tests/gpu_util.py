"""Helpers of the GPU parity tests: oracle states <-> device tensors."""
from __future__ import annotations

import numpy as np
import torch

from oracle import numerics as nm
from oracle import sim
from krea2_svdquant_amd import SVDQuantLinearState


def bf16_tensor(a: np.ndarray, dev) -> torch.Tensor:
    """float32 array of bf16 values (or uint16 bits) -> torch bf16 tensor on dev."""
    bits = a if a.dtype == np.uint16 else nm.bf16_bits(a)
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def bf16_bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_device_state(st: sim.LayerState, dev) -> SVDQuantLinearState:
    return SVDQuantLinearState(
        smooth_scale=bf16_tensor(st.smooth, dev),
        qweight=torch.from_numpy(np.ascontiguousarray(st.qweight)).to(dev),
        weight_scales=torch.from_numpy(st.weight_scales.astype(np.float16)).to(dev),
        l1=bf16_tensor(st.l1, dev), l2=bf16_tensor(st.l2, dev),
        bias=None if st.bias is None else bf16_tensor(st.bias, dev),
        group_size=st.group_size, original_shape=st.shape, qweight_packed=True,
        padded_in_features=st.padded_in)


class _Adapter:
    def __init__(self, ad: sim.Adapter, dev):
        self.down_weight = bf16_tensor(ad.down, dev)
        self.up_weight = bf16_tensor(ad.up, dev)
        self.multiplier = ad.multiplier


def device_adapters(st: sim.LayerState, dev):
    return [_Adapter(a, dev) for a in st.adapters]


def from_device_state(ds: SVDQuantLinearState) -> sim.LayerState:
    """A device state (e.g. built by the converter on the GPU) as an oracle state."""
    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    return sim.LayerState(smooth=f(ds.smooth_scale), qweight=ds.qweight.cpu().numpy(),
                          weight_scales=f(ds.weight_scales), l1=f(ds.l1), l2=f(ds.l2),
                          bias=None if ds.bias is None else f(ds.bias), group_size=ds.group_size,
                          shape=tuple(ds.original_shape))


PERM8 = [0, 2, 4, 6, 1, 3, 5, 7]
"""GEMM operand byte order inside each chunk of 8 columns: byte j holds column PERM8[j]."""


def operand_bytes(q: np.ndarray, fmt: str) -> np.ndarray:
    """Expected W4A4 operand codes [M, K] for int codes q: OCP e4m3 (torch's float8_e4m3fn
    encoder) or int8 16*q, in the PERM8 byte order."""
    m, k = q.shape
    if fmt == "e4m3":
        codes = torch.from_numpy(q.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    else:
        codes = (q.astype(np.int16) * 16).astype(np.int8).view(np.uint8)
    return codes.reshape(m, k // 8, 8)[:, :, PERM8].reshape(m, k)


def rel_l2(a, b) -> float:
    return sim.rel_l2(a, b)
