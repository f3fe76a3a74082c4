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


def e3m2_code(q: np.ndarray) -> np.ndarray:
    """6-bit e3m2 (OCP FP6 "bf6": sign, 3 exponent bits with bias 3, 2 mantissa bits) codes of
    integers q in [-8, 7], from the format definition: |q| = 2^e (1 + m/4), code = s<<5 | (e+3)<<2 | m."""
    q = np.asarray(q, np.int64)
    a = np.abs(q)
    e = np.floor(np.log2(np.maximum(a, 1))).astype(np.int64)
    m = np.rint((a / 2.0 ** e - 1.0) * 4).astype(np.int64)
    mag = np.where(a == 0, 0, ((e + 3) << 2) | m)
    return (mag | ((q < 0).astype(np.int64) << 5)).astype(np.uint8)


def e3m2_value(code: np.ndarray) -> np.ndarray:
    """Decode 6-bit e3m2 codes (normal: 2^(E-3) (1 + M/4); subnormal E = 0: 2^-2 M/4)."""
    c = np.asarray(code, np.int64)
    s, ex, mt = (c >> 5) & 1, (c >> 2) & 7, c & 3
    v = np.where(ex == 0, mt / 4.0 * 2.0 ** -2, (1 + mt / 4.0) * 2.0 ** (ex - 3))
    return np.where(s == 1, -v, v)


def e3m2_planar(q: np.ndarray) -> np.ndarray:
    """Flat planar e3m2 operand bytes of int codes q [R, K] (the layout of svdq_act_quant's e3m2
    qa): per k-step t and half h the 32 codes of a row are contiguous little-endian 6-bit fields
    (field f = column 64 t + 32 h + f) in 24 bytes, bytes 0-15 in plane Q[t][h][Rp][16], bytes
    16-23 in plane P[t][h][Rp][8] after all Q planes; Rp = R rounded up to even, padding zero."""
    r, k = q.shape
    rp, t = (r + 1) & ~1, k // 64
    c = e3m2_code(q).astype(np.uint8).reshape(r, t, 2, 32)
    bits = np.zeros((r, t, 2, 192), np.uint8)
    for b in range(6):
        bits[..., np.arange(32) * 6 + b] = (c >> b) & 1
    v24 = np.packbits(bits.reshape(r, t, 2, 24, 8), axis=-1, bitorder="little").reshape(r, t, 2, 24)
    qp = np.zeros((t, 2, rp, 16), np.uint8)
    pp = np.zeros((t, 2, rp, 8), np.uint8)
    qp[:, :, :r] = v24[..., :16].transpose(1, 2, 0, 3)
    pp[:, :, :r] = v24[..., 16:].transpose(1, 2, 0, 3)
    return np.concatenate([qp.ravel(), pp.ravel()])


def e3m2_rows(buf: np.ndarray, r: int, k: int) -> np.ndarray:
    """The written rows of a flat planar e3m2 operand as [K/64, 2, R, 24] (padding rows dropped)."""
    rp, t = (r + 1) & ~1, k // 64
    buf = np.asarray(buf, np.uint8).ravel()
    qp = buf[:t * 2 * rp * 16].reshape(t, 2, rp, 16)[:, :, :r]
    pp = buf[t * 2 * rp * 16:].reshape(t, 2, rp, 8)[:, :, :r]
    return np.concatenate([qp, pp], axis=-1)


def e3m2_codes_of(buf: np.ndarray, r: int, k: int, rows=None) -> np.ndarray:
    """Integer codes [R', K] decoded from a flat planar e3m2 operand (the inverse of e3m2_planar,
    through the format's own decoding e3m2_value), for all rows or the listed ``rows``.  Each
    3-byte run of a row's 24 bytes holds 4 little-endian 6-bit fields."""
    v24 = e3m2_rows(buf, r, k)                       # [K/64, 2, R, 24]
    if rows is not None:
        v24 = v24[:, :, np.asarray(rows)]
    b = v24.reshape(*v24.shape[:3], 8, 3).astype(np.uint32)
    u = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)              # [K/64, 2, R', 8]
    fields = np.stack([(u >> (6 * i)) & 63 for i in range(4)], axis=-1).reshape(*u.shape[:3], 32)
    vals = e3m2_value(np.arange(64))
    exact = (vals == np.rint(vals)) & (vals >= -8) & (vals <= 7)
    table = np.where(exact, np.rint(vals), 99).astype(np.int8)    # 99: not an INT4 code
    t = k // 64
    return table[fields].transpose(2, 0, 1, 3).reshape(-1, t * 64)


def sx_pairs_ok(sx_pairs: torch.Tensor, sx_ref: np.ndarray, rows=None) -> bool:
    """sx pairs [K/G, M] (u32 bf16 | bf16 << 16) against the oracle's bf16 scales [M, K/G]."""
    got = sx_pairs.cpu().numpy().view(np.uint32).T
    if rows is not None:
        got = got[np.asarray(rows)]
    bits = nm.bf16_bits(sx_ref).astype(np.uint32)
    return bool(np.array_equal(got, bits | (bits << 16)))
