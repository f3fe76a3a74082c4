"""torch custom ops ``svdq::*`` over the gfx950 C-ABI.

Each op validates dtype / device / shape / contiguity, allocates its outputs with the torch
caching allocator on the input's device, and enqueues the C-ABI call on the current HIP
stream (no host synchronisation).  Fake (meta) implementations describe the output shapes.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import lib

_counters: dict[tuple[int, int], Tensor] = {}


def _vp(t: Optional[Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(cond: bool, exc, msg: str) -> None:
    if not cond:
        raise exc(msg)


def _check_dev(name: str, t: Tensor, device: torch.device, dtype: torch.dtype) -> None:
    _need(t.device == device, ValueError, f"{name} is on {t.device}, expected {device}")
    _need(t.dtype == dtype, TypeError, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), ValueError, f"{name} must be contiguous")


def _arrival_counters(device: torch.device, n: int) -> Tensor:
    """Zero-initialised arrival counters of the split reduction (per device and stream).

    The kernel leaves them zero after every completed launch, so they are allocated once.
    """
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    buf = _counters.get(key)
    if buf is None or buf.numel() < n:
        buf = torch.zeros(max(n, 64), dtype=torch.int32, device=device)
        _counters[key] = buf
    return buf


def rank_padded(total_rank: int) -> int:
    """Row stride of ``mid`` / ``l1cat``: rank + LoRA rank rounded up to 32."""
    return max(32, (total_rank + 31) // 32 * 32)


@torch.library.custom_op("svdq::prepare_smooth", mutates_args=())
def prepare_smooth(smooth: Tensor) -> Tensor:
    """[2K] float32: float(smooth) then RN(1 / float(smooth)), for ``svdq::act_quant``."""
    _need(smooth.is_cuda, RuntimeError, "svdq::prepare_smooth needs a GPU tensor")
    _check_dev("smooth", smooth, smooth.device, torch.bfloat16)
    k = smooth.numel()
    srs = torch.empty(2 * k, dtype=torch.float32, device=smooth.device)
    lib.call("svdq_prepare_smooth", _vp(smooth), _vp(srs), k, _stream(smooth.device))
    return srs


@prepare_smooth.register_fake
def _(smooth):
    return smooth.new_empty(2 * smooth.numel(), dtype=torch.float32)


@torch.library.custom_op("svdq::act_quant", mutates_args=())
def act_quant(x: Tensor, srs: Tensor, l2: Tensor, lora_down: Optional[Tensor],
              lora_mult: Optional[Tensor], group_size: int, rtp: int, quant: bool, want_xhat: bool,
              exact: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Smoothing + A4 quantization + packing + low-rank / LoRA down projections, one pass.

    Returns ``(qx uint8 [M, K/2], sx bf16 [M, K/G], xhat bf16 [M, K], mid f32 [M, rtp])``;
    outputs not requested (``quant`` / ``want_xhat``) are empty tensors.
    """
    _need(x.is_cuda, RuntimeError, "svdq::act_quant needs a GPU tensor")
    dev = x.device
    _need(x.dim() == 2, ValueError, f"x must be 2-D [M, K], got {tuple(x.shape)}")
    _check_dev("x", x, dev, torch.bfloat16)
    m, k = x.shape
    _check_dev("srs", srs, dev, torch.float32)
    _need(srs.numel() == 2 * k, ValueError, f"srs has {srs.numel()} elements, expected {2 * k}")
    _check_dev("l2", l2, dev, torch.bfloat16)
    _need(l2.dim() == 2 and l2.shape[1] == k, ValueError, f"l2 must be [r, {k}], got {tuple(l2.shape)}")
    r = l2.shape[0]
    rl = 0
    if lora_down is not None:
        _check_dev("lora_down", lora_down, dev, torch.bfloat16)
        _need(lora_down.dim() == 2 and lora_down.shape[1] == k, ValueError,
              f"lora_down must be [rl, {k}], got {tuple(lora_down.shape)}")
        rl = lora_down.shape[0]
        _need(lora_mult is not None and lora_mult.numel() == rl, ValueError, "lora_mult must have rl entries")
        _check_dev("lora_mult", lora_mult, dev, torch.float32)
    _need(k % group_size == 0, ValueError, f"K={k} must be a multiple of group_size={group_size}")

    splits = ctypes.c_int()
    midp_n = ctypes.c_int64()
    cnt_n = ctypes.c_int64()
    lib.call("svdq_act_quant_workspace", m, k, group_size, rtp, ctypes.byref(splits),
             ctypes.byref(midp_n), ctypes.byref(cnt_n))
    qx = torch.empty((m, k // 2) if quant else (0,), dtype=torch.uint8, device=dev)
    sx = torch.empty((m, k // group_size) if quant else (0,), dtype=torch.bfloat16, device=dev)
    xhat = torch.empty((m, k) if want_xhat else (0,), dtype=torch.bfloat16, device=dev)
    mid = torch.empty((m, rtp), dtype=torch.float32, device=dev)
    midp = torch.empty(midp_n.value, dtype=torch.float32, device=dev) if midp_n.value else None
    counters = _arrival_counters(dev, cnt_n.value) if splits.value > 1 else None
    flags = ((lib.SVDQ_ACT_QUANT if quant else 0) | (lib.SVDQ_ACT_XHAT if want_xhat else 0)
             | (lib.SVDQ_ACT_EXACT_DIV if exact else 0))
    lib.call("svdq_act_quant", _vp(x), k, _vp(srs), _vp(l2), r, _vp(lora_down), rl, _vp(lora_mult),
             m, k, group_size, rtp, flags, _vp(qx) if quant else None, _vp(sx) if quant else None,
             _vp(xhat) if want_xhat else None, k, _vp(mid), _vp(midp), _vp(counters), splits.value,
             _stream(dev))
    return qx, sx, xhat, mid


@act_quant.register_fake
def _(x, srs, l2, lora_down, lora_mult, group_size, rtp, quant, want_xhat, exact):
    m, k = x.shape
    qx = x.new_empty((m, k // 2) if quant else (0,), dtype=torch.uint8)
    sx = x.new_empty((m, k // group_size) if quant else (0,), dtype=torch.bfloat16)
    xhat = x.new_empty((m, k) if want_xhat else (0,), dtype=torch.bfloat16)
    return qx, sx, xhat, x.new_empty((m, rtp), dtype=torch.float32)


def _check_gemm(qweight: Tensor, weight_scales: Tensor, mid: Tensor, l1cat: Tensor, bias: Optional[Tensor],
                m: int, k: int, group_size: int, dev: torch.device) -> int:
    _check_dev("qweight", qweight, dev, torch.uint8)
    _need(qweight.dim() == 2 and qweight.shape[1] * 2 == k, ValueError,
          f"qweight must be [N, {k // 2}], got {tuple(qweight.shape)}")
    n = qweight.shape[0]
    _check_dev("weight_scales", weight_scales, dev, torch.float16)
    _need(tuple(weight_scales.shape) == (n, k // group_size), ValueError,
          f"weight_scales must be [{n}, {k // group_size}], got {tuple(weight_scales.shape)}")
    _check_dev("mid", mid, dev, torch.float32)
    _need(mid.dim() == 2 and mid.shape[0] == m, ValueError, f"mid must be [{m}, RTp]")
    _check_dev("l1cat", l1cat, dev, torch.bfloat16)
    _need(tuple(l1cat.shape) == (n, mid.shape[1]), ValueError,
          f"l1cat must be [{n}, {mid.shape[1]}], got {tuple(l1cat.shape)}")
    if bias is not None:
        _check_dev("bias", bias, dev, torch.bfloat16)
        _need(bias.numel() == n, ValueError, f"bias must have {n} entries")
    return n


@torch.library.custom_op("svdq::w4a4_gemm", mutates_args=())
def w4a4_gemm(qx: Tensor, sx: Tensor, qweight: Tensor, weight_scales: Tensor, mid: Tensor, l1cat: Tensor,
              bias: Optional[Tensor], group_size: int, out_f32: bool) -> Tensor:
    """``y = sum_g sx sw (qx . qw)_g + mid @ l1cat^T + bias`` (bf16 or float32 output)."""
    _need(qx.is_cuda, RuntimeError, "svdq::w4a4_gemm needs GPU tensors")
    dev = qx.device
    _check_dev("qx", qx, dev, torch.uint8)
    m, k = qx.shape[0], qx.shape[1] * 2
    _check_dev("sx", sx, dev, torch.bfloat16)
    _need(tuple(sx.shape) == (m, k // group_size), ValueError, "sx must be [M, K/G]")
    n = _check_gemm(qweight, weight_scales, mid, l1cat, bias, m, k, group_size, dev)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    lib.call("svdq_w4a4_gemm", _vp(qx), _vp(sx), _vp(qweight), _vp(weight_scales), _vp(mid), _vp(l1cat),
             mid.shape[1], _vp(bias), m, n, k, group_size, _vp(y), n, int(out_f32), _stream(dev))
    return y


@w4a4_gemm.register_fake
def _(qx, sx, qweight, weight_scales, mid, l1cat, bias, group_size, out_f32):
    return qx.new_empty((qx.shape[0], qweight.shape[0]), dtype=torch.float32 if out_f32 else torch.bfloat16)


@torch.library.custom_op("svdq::w4a16_gemm", mutates_args=())
def w4a16_gemm(xhat: Tensor, qweight: Tensor, weight_scales: Tensor, mid: Tensor, l1cat: Tensor,
               bias: Optional[Tensor], group_size: int, out_f32: bool) -> Tensor:
    """``y = xhat @ bf16(q * bf16(sw))^T + mid @ l1cat^T + bias`` (bf16 or float32 output)."""
    _need(xhat.is_cuda, RuntimeError, "svdq::w4a16_gemm needs GPU tensors")
    dev = xhat.device
    _check_dev("xhat", xhat, dev, torch.bfloat16)
    m, k = xhat.shape
    n = _check_gemm(qweight, weight_scales, mid, l1cat, bias, m, k, group_size, dev)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    lib.call("svdq_w4a16_gemm", _vp(xhat), k, _vp(qweight), _vp(weight_scales), _vp(mid), _vp(l1cat),
             mid.shape[1], _vp(bias), m, n, k, group_size, _vp(y), n, int(out_f32), _stream(dev))
    return y


@w4a16_gemm.register_fake
def _(xhat, qweight, weight_scales, mid, l1cat, bias, group_size, out_f32):
    return xhat.new_empty((xhat.shape[0], qweight.shape[0]), dtype=torch.float32 if out_f32 else torch.bfloat16)
