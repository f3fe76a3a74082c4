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


OPERAND_NONE, OPERAND_E4M3, OPERAND_I8, OPERAND_E3M2 = -1, 0, 1, 2
_OPERANDS = (OPERAND_E4M3, OPERAND_I8, OPERAND_E3M2)


def operand_bytes(rows: int, k: int, operand: int) -> int:
    """Bytes of an [rows, K] W4A4 operand in format ``operand``: one per code for e4m3 / int8; the
    planar e3m2 layout holds 6 bits per code with rows padded to an even count."""
    return ((rows + 1) & ~1) * k * 3 // 4 if operand == OPERAND_E3M2 else rows * k


def _operand_shape(rows: int, k: int, operand: int) -> tuple:
    return (operand_bytes(rows, k, operand),) if operand == OPERAND_E3M2 else (rows, k)


@torch.library.custom_op("svdq::prepare_weight_scales", mutates_args=())
def prepare_weight_scales(weight_scales: Tensor, operand: int) -> Tensor:
    """[K/G, N] uint32 (bf16 hi | bf16 lo << 16) operand of the W4A4 scale MFMA, per layer
    (group-major: the transpose of the checkpoint's [N, K/G] fp16 ``weight_scales``)."""
    _need(weight_scales.is_cuda, RuntimeError, "svdq::prepare_weight_scales needs a GPU tensor")
    _check_dev("weight_scales", weight_scales, weight_scales.device, torch.float16)
    _need(weight_scales.dim() == 2, ValueError, f"weight_scales must be [N, K/G], got {tuple(weight_scales.shape)}")
    _need(operand in _OPERANDS, ValueError, f"operand={operand}")
    n, ng = weight_scales.shape
    out = torch.empty((ng, n), dtype=torch.int32, device=weight_scales.device)
    lib.call("svdq_prepare_weight_scales", _vp(weight_scales), _vp(out), n, ng, operand, _stream(weight_scales.device))
    return out


@prepare_weight_scales.register_fake
def _(weight_scales, operand):
    return weight_scales.new_empty((weight_scales.shape[1], weight_scales.shape[0]), dtype=torch.int32)


@torch.library.custom_op("svdq::prepare_weight_operand", mutates_args=())
def prepare_weight_operand(qweight: Tensor, operand: int) -> Tensor:
    """W4A4 weight operand, per layer: the packed INT4 codes [N, K/2] as MFMA operand codes in the
    layout and format of ``act_quant``'s ``qa``: uint8 [N, K] for e4m3 / int8, the flat planar
    e3m2 bytes (``operand_bytes(N, K, OPERAND_E3M2)``) for e3m2."""
    _need(qweight.is_cuda, RuntimeError, "svdq::prepare_weight_operand needs a GPU tensor")
    _check_dev("qweight", qweight, qweight.device, torch.uint8)
    _need(qweight.dim() == 2, ValueError, f"qweight must be [N, K/2], got {tuple(qweight.shape)}")
    _need(operand in _OPERANDS, ValueError, f"operand={operand}")
    n, k = qweight.shape[0], qweight.shape[1] * 2
    out = torch.empty(_operand_shape(n, k, operand), dtype=torch.uint8, device=qweight.device)
    lib.call("svdq_prepare_weight_operand", _vp(qweight), _vp(out), n, k, operand, _stream(qweight.device))
    return out


@prepare_weight_operand.register_fake
def _(qweight, operand):
    return qweight.new_empty(_operand_shape(qweight.shape[0], qweight.shape[1] * 2, operand), dtype=torch.uint8)


OPERAND_NAMES = {"e4m3": OPERAND_E4M3, "fp8": OPERAND_E4M3, "i8": OPERAND_I8, "int8": OPERAND_I8,
                 "e3m2": OPERAND_E3M2, "fp6": OPERAND_E3M2}


@torch.library.custom_op("svdq::act_quant", mutates_args=())
def act_quant(x: Tensor, srs: Tensor, l2: Tensor, lora_down: Optional[Tensor],
              lora_mult: Optional[Tensor], group_size: int, rtp: int, operand: int, packed: bool,
              want_xhat: bool, exact: bool, sx_pairs: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Smoothing + A4 quantization + low-rank / LoRA down projections, one pass over x.

    ``operand`` selects the W4A4 GEMM operand codes written (``OPERAND_E4M3`` / ``OPERAND_I8`` /
    ``OPERAND_E3M2``, the last in the flat planar layout) or none (``OPERAND_NONE``: x_hat only,
    the W4A16 path).  Returns
    ``(qa uint8 [M, K], sx bf16 [M, K/G], qx uint8 [M, K/2], xhat bf16 [M, K], mid f32 [S + 1, M, rtp])``
    where ``mid`` is the pass's workspace: ``mid[0]`` holds the GEMM epilogue operand (bf16 hi and
    lo planes per row, see ``mid_values``), ``mid[1:]`` one partial per K split; outputs not
    requested are empty tensors (``qx`` needs ``packed``, ``xhat`` ``want_xhat``).  With ``sx_pairs`` the
    scales come as int32 [K/G, M] (group-major) bf16 pairs (bits | bits << 16), the form
    ``w4a4_gemm`` takes.
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
    _need(operand == OPERAND_NONE or operand in _OPERANDS, ValueError, f"operand={operand}")
    quant = operand != OPERAND_NONE
    _need(quant or not sx_pairs, ValueError, "sx_pairs needs an operand format")

    splits = _splits(m, k, group_size, rtp)
    qa = torch.empty(_operand_shape(m, k, operand) if quant else (0,), dtype=torch.uint8, device=dev)
    sx_shape = ((k // group_size, m) if sx_pairs else (m, k // group_size)) if quant else (0,)
    sx = torch.empty(sx_shape, dtype=torch.int32 if sx_pairs else torch.bfloat16, device=dev)
    qx = torch.empty((m, k // 2) if packed else (0,), dtype=torch.uint8, device=dev)
    xhat = torch.empty((m, k) if want_xhat else (0,), dtype=torch.bfloat16, device=dev)
    mid = torch.empty((splits + 1, m, rtp), dtype=torch.float32, device=dev)
    flags = ((lib.SVDQ_ACT_OPERAND_E4M3 if operand == OPERAND_E4M3 else 0)
             | (lib.SVDQ_ACT_OPERAND_I8 if operand == OPERAND_I8 else 0)
             | (lib.SVDQ_ACT_OPERAND_E3M2 if operand == OPERAND_E3M2 else 0)
             | (lib.SVDQ_ACT_PACKED if packed else 0) | (lib.SVDQ_ACT_XHAT if want_xhat else 0)
             | (lib.SVDQ_ACT_EXACT_DIV if exact else 0) | (lib.SVDQ_ACT_SX_PAIRS if sx_pairs else 0))
    lib.call("svdq_act_quant", _vp(x), k, _vp(srs), _vp(l2), r, _vp(lora_down), rl, _vp(lora_mult),
             m, k, group_size, rtp, flags, _vp(qa) if quant else None, _vp(sx) if quant else None,
             _vp(qx) if packed else None, _vp(xhat) if want_xhat else None, k, _vp(mid), splits,
             _stream(dev))
    return qa, sx, qx, xhat, mid


@act_quant.register_fake
def _(x, srs, l2, lora_down, lora_mult, group_size, rtp, operand, packed, want_xhat, exact, sx_pairs=False):
    m, k = x.shape
    quant = operand != OPERAND_NONE
    qa = x.new_empty(_operand_shape(m, k, operand) if quant else (0,), dtype=torch.uint8)
    sx_shape = ((k // group_size, m) if sx_pairs else (m, k // group_size)) if quant else (0,)
    sx = x.new_empty(sx_shape, dtype=torch.int32 if sx_pairs else torch.bfloat16)
    qx = x.new_empty((m, k // 2) if packed else (0,), dtype=torch.uint8)
    xhat = x.new_empty((m, k) if want_xhat else (0,), dtype=torch.bfloat16)
    return qa, sx, qx, xhat, x.new_empty((_splits(m, k, group_size, rtp) + 1, m, rtp), dtype=torch.float32)


_split_cache: dict[tuple[int, int, int, int], int] = {}


@torch.library.custom_op("svdq::act_quant_siblings", mutates_args=())
def act_quant_siblings(x: Tensor, srs: list[Tensor], l2: list[Tensor], group_size: int, rtp: int,
                       exact: bool) -> list[Tensor]:
    """``act_quant(x, srs[i], l2[i], None, None, group_size, rtp, OPERAND_E3M2, False, False, exact,
    True)`` for sibling layers i over the same x (no LoRA), as one launch when every rank is at most
    32 and the group 64 or 128 (``svdq_act_quant_siblings``).  Returns ``[qa_0, sx_0, mid_0, qa_1,
    ...]``, each bit-identical to that layer's ``act_quant``."""
    _need(x.is_cuda, RuntimeError, "svdq::act_quant_siblings needs a GPU tensor")
    count = len(srs)
    _need(1 <= count <= lib.SVDQ_MAX_SIBLINGS and len(l2) == count, ValueError,
          f"1..{lib.SVDQ_MAX_SIBLINGS} layers with one srs and one l2 each")
    dev = x.device
    _need(x.dim() == 2, ValueError, f"x must be 2-D [M, K], got {tuple(x.shape)}")
    _check_dev("x", x, dev, torch.bfloat16)
    m, k = x.shape
    _need(k % group_size == 0, ValueError, f"K={k} must be a multiple of group_size={group_size}")
    for i in range(count):
        _check_dev(f"srs[{i}]", srs[i], dev, torch.float32)
        _need(srs[i].numel() == 2 * k, ValueError, f"srs[{i}] has {srs[i].numel()} elements, expected {2 * k}")
        _check_dev(f"l2[{i}]", l2[i], dev, torch.bfloat16)
        _need(l2[i].dim() == 2 and l2[i].shape[1] == k, ValueError, f"l2[{i}] must be [r, {k}]")
    splits = _splits(m, k, group_size, rtp)
    outs, arr = [], (lib.ActSibling * count)()
    for i in range(count):
        qa = torch.empty(_operand_shape(m, k, OPERAND_E3M2), dtype=torch.uint8, device=dev)
        sx = torch.empty((k // group_size, m), dtype=torch.int32, device=dev)
        mid = torch.empty((splits + 1, m, rtp), dtype=torch.float32, device=dev)
        arr[i] = lib.ActSibling(srs[i].data_ptr(), l2[i].data_ptr(), l2[i].shape[0], qa.data_ptr(), sx.data_ptr(),
                                mid.data_ptr())
        outs += [qa, sx, mid]
    flags = lib.SVDQ_ACT_OPERAND_E3M2 | lib.SVDQ_ACT_SX_PAIRS | (lib.SVDQ_ACT_EXACT_DIV if exact else 0)
    lib.call("svdq_act_quant_siblings", _vp(x), k, arr, count, m, k, group_size, rtp, flags, splits, _stream(dev))
    return outs


@act_quant_siblings.register_fake
def _(x, srs, l2, group_size, rtp, exact):
    m, k = x.shape
    splits = _splits(m, k, group_size, rtp)
    out = []
    for _i in range(len(srs)):
        out += [x.new_empty(_operand_shape(m, k, OPERAND_E3M2), dtype=torch.uint8),
                x.new_empty((k // group_size, m), dtype=torch.int32),
                x.new_empty((splits + 1, m, rtp), dtype=torch.float32)]
    return out


def _splits(m: int, k: int, group_size: int, rtp: int) -> int:
    """Number of K splits the activation pass uses for this shape (leading dim of ``mid``)."""
    key = (m, k, group_size, rtp)
    hit = _split_cache.get(key)
    if hit is None:
        splits, mid_n = ctypes.c_int(), ctypes.c_int64()
        lib.call("svdq_act_quant_workspace", m, k, group_size, rtp, ctypes.byref(splits), ctypes.byref(mid_n))
        hit = _split_cache[key] = splits.value
    return hit


def mid_values(mid: Tensor) -> Tensor:
    """The low-rank activations ``act_quant`` left at the head of its ``mid`` workspace, as float32
    [M, rtp]: the bf16 hi plane plus the bf16 lo plane of each row."""
    m, rtp = mid.shape[1], mid.shape[2]
    planes = mid[0].contiguous().view(torch.bfloat16).view(m, 2, rtp).float()
    return planes[:, 0] + planes[:, 1]


def pack_mid(values: Tensor) -> Tensor:
    """Inverse of ``mid_values`` for a float32 [M, rtp] tensor: a [1, M, rtp] workspace whose head
    holds the hi / lo planes the GEMMs read (hi = bf16(v), lo = bf16(v - hi))."""
    v = values.float().contiguous()
    hi = v.to(torch.bfloat16)
    lo = (v - hi.float()).to(torch.bfloat16)
    return torch.stack((hi, lo), dim=1).contiguous().view(torch.float32).view(1, v.shape[0], v.shape[1])


def _check_epilogue(mid: Tensor, l1cat: Tensor, bias: Optional[Tensor], m: int, n: int, dev: torch.device) -> None:
    _check_dev("mid", mid, dev, torch.float32)
    _need(mid.dim() == 3 and mid.shape[0] >= 1 and mid.shape[1] == m, ValueError,
          f"mid must be act_quant's workspace [S + 1, {m}, RTp]")
    _check_dev("l1cat", l1cat, dev, torch.bfloat16)
    _need(tuple(l1cat.shape) == (n, mid.shape[2]), ValueError,
          f"l1cat must be [{n}, {mid.shape[2]}], got {tuple(l1cat.shape)}")
    if bias is not None:
        _check_dev("bias", bias, dev, torch.bfloat16)
        _need(bias.numel() == n, ValueError, f"bias must have {n} entries")


def _check_gemm(qweight: Tensor, weight_scales: Tensor, mid: Tensor, l1cat: Tensor, bias: Optional[Tensor],
                m: int, k: int, group_size: int, dev: torch.device) -> int:
    _check_dev("qweight", qweight, dev, torch.uint8)
    _need(qweight.dim() == 2 and qweight.shape[1] * 2 == k, ValueError,
          f"qweight must be [N, {k // 2}], got {tuple(qweight.shape)}")
    n = qweight.shape[0]
    _check_dev("weight_scales", weight_scales, dev, torch.float16)
    _need(tuple(weight_scales.shape) == (n, k // group_size), ValueError,
          f"weight_scales must be [{n}, {k // group_size}], got {tuple(weight_scales.shape)}")
    _check_epilogue(mid, l1cat, bias, m, n, dev)
    return n


EPILOGUES = {"none": lib.SVDQ_EPI_NONE, "mul_sigmoid": lib.SVDQ_EPI_MUL_SIGMOID,
             "silu_mul": lib.SVDQ_EPI_SILU_MUL, "residual_gate": lib.SVDQ_EPI_RESIDUAL_GATE}


def _check_epi(epi: int, aux: Optional[Tensor], vec: Optional[Tensor], m: int, n: int, out_f32: bool,
               dev: torch.device) -> None:
    """Validate the operands of a fused epilogue op (``EPILOGUES``)."""
    _need(epi in EPILOGUES.values(), ValueError, f"epilogue op {epi}")
    if epi == lib.SVDQ_EPI_NONE:
        _need(aux is None and vec is None, ValueError, "aux / vec given without an epilogue op")
        return
    _need(not out_f32, ValueError, "epilogue ops need bf16 output")
    _need(aux is not None, ValueError, "epilogue op needs aux")
    _check_dev("aux", aux, dev, torch.bfloat16)
    _need(tuple(aux.shape) == (m, n), ValueError, f"aux must be [{m}, {n}], got {tuple(aux.shape)}")
    if epi == lib.SVDQ_EPI_RESIDUAL_GATE:
        _need(vec is not None, ValueError, "residual_gate needs vec")
        _check_dev("vec", vec, dev, torch.bfloat16)
        _need(vec.numel() == n, ValueError, f"vec must have {n} entries")
    else:
        _need(vec is None, ValueError, "vec is only used by residual_gate")


def _epi_args(epi: int, aux: Optional[Tensor], vec: Optional[Tensor], n: int) -> tuple:
    return (epi, _vp(aux), aux.shape[1] if aux is not None else n, _vp(vec))


@torch.library.custom_op("svdq::w4a4_gemm", mutates_args=())
def w4a4_gemm(qa: Tensor, sx_pairs: Tensor, weight_operand: Tensor, weight_scale_pairs: Tensor, mid: Tensor,
              l1cat: Tensor, bias: Optional[Tensor], group_size: int, operand: int, out_f32: bool,
              epi: int = 0, aux: Optional[Tensor] = None, vec: Optional[Tensor] = None) -> Tensor:
    """``y = sum_g sx sw (qa . qw)_g + mid @ l1cat^T + bias`` (bf16 or float32 output), then the
    elementwise op ``epi`` (``EPILOGUES``; bf16 output) with ``aux`` [M, N] and ``vec`` [N].

    ``sx_pairs`` comes from ``act_quant(..., sx_pairs=True)``; ``weight_operand`` and
    ``weight_scale_pairs`` from ``prepare_weight_operand`` and ``prepare_weight_scales`` with
    the same ``operand``.
    """
    _need(qa.is_cuda, RuntimeError, "svdq::w4a4_gemm needs GPU tensors")
    dev = qa.device
    _need(operand in _OPERANDS, ValueError, f"operand={operand}")
    m, n, k = _check_w4a4_operands(qa, sx_pairs, weight_operand, weight_scale_pairs, mid, l1cat, bias, group_size,
                                   operand, dev)
    _check_epi(epi, aux, vec, m, n, out_f32, dev)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    lib.call("svdq_w4a4_gemm_epi", _vp(qa), operand, _vp(sx_pairs), _vp(weight_operand), _vp(weight_scale_pairs),
             _vp(mid), _vp(l1cat), mid.shape[2], _vp(bias), m, n, k, group_size, _vp(y), n, int(out_f32),
             *_epi_args(epi, aux, vec, n), _stream(dev))
    return y


@w4a4_gemm.register_fake
def _(qa, sx_pairs, weight_operand, weight_scale_pairs, mid, l1cat, bias, group_size, operand, out_f32,
      epi=0, aux=None, vec=None):
    return qa.new_empty((sx_pairs.shape[1], weight_scale_pairs.shape[1]),
                        dtype=torch.float32 if out_f32 else torch.bfloat16)


def _check_w4a4_operands(qa: Tensor, sx_pairs: Tensor, weight_operand: Tensor, weight_scale_pairs: Tensor,
                         mid: Tensor, l1cat: Tensor, bias: Optional[Tensor], group_size: int, operand: int,
                         dev: torch.device, who: str = "") -> tuple[int, int, int]:
    """Checks of one W4A4 layer's GEMM operands; returns (M, N, K)."""
    _check_dev(f"{who}qa", qa, dev, torch.uint8)
    _check_dev(f"{who}sx_pairs", sx_pairs, dev, torch.int32)
    _need(sx_pairs.dim() == 2, ValueError, f"{who}sx_pairs must be [K/G, M]")
    m, k = sx_pairs.shape[1], sx_pairs.shape[0] * group_size
    _need(tuple(qa.shape) == _operand_shape(m, k, operand), ValueError,
          f"{who}qa must be {_operand_shape(m, k, operand)} for M={m}, K={k}, got {tuple(qa.shape)}")
    _check_dev(f"{who}weight_operand", weight_operand, dev, torch.uint8)
    _check_dev(f"{who}weight_scale_pairs", weight_scale_pairs, dev, torch.int32)
    _need(weight_scale_pairs.dim() == 2 and weight_scale_pairs.shape[0] == k // group_size, ValueError,
          f"{who}weight_scale_pairs must be [{k // group_size}, N], got {tuple(weight_scale_pairs.shape)}")
    n = weight_scale_pairs.shape[1]
    _need(tuple(weight_operand.shape) == _operand_shape(n, k, operand), ValueError,
          f"{who}weight_operand must be {_operand_shape(n, k, operand)}, got {tuple(weight_operand.shape)}")
    _check_epilogue(mid, l1cat, bias, m, n, dev)
    return m, n, k


@torch.library.custom_op("svdq::w4a4_gemm_siblings", mutates_args=())
def w4a4_gemm_siblings(qa: list[Tensor], sx_pairs: list[Tensor], weight_operand: list[Tensor],
                       weight_scale_pairs: list[Tensor], mid: list[Tensor], l1cat: list[Tensor],
                       bias: list[Optional[Tensor]], group_size: int, operand: int, out_f32: bool) -> list[Tensor]:
    """``w4a4_gemm`` of up to ``lib.SVDQ_MAX_SIBLINGS`` layers over the same rows (the i-th entry
    of every list belongs to layer i), in one launch (``svdq_w4a4_gemm_siblings``); each output is
    bit-identical to that layer's ``w4a4_gemm``."""
    count = len(qa)
    _need(1 <= count <= lib.SVDQ_MAX_SIBLINGS, ValueError, f"1..{lib.SVDQ_MAX_SIBLINGS} layers, got {count}")
    _need(all(len(a) == count for a in (sx_pairs, weight_operand, weight_scale_pairs, mid, l1cat, bias)),
          ValueError, "one entry per layer in every list")
    _need(qa[0].is_cuda, RuntimeError, "svdq::w4a4_gemm_siblings needs GPU tensors")
    _need(operand in _OPERANDS, ValueError, f"operand={operand}")
    dev = qa[0].device
    shapes = [_check_w4a4_operands(qa[i], sx_pairs[i], weight_operand[i], weight_scale_pairs[i], mid[i], l1cat[i],
                                   bias[i], group_size, operand, dev, f"layer {i}: ") for i in range(count)]
    m, _, k = shapes[0]
    _need(all(s[0] == m and s[2] == k for s in shapes), ValueError,
          f"sibling layers need the same M and K, got {[(s[0], s[2]) for s in shapes]}")
    ys = [torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev) for _, n, _ in shapes]
    arr = (lib.W4A4Sibling * count)()
    for i, (y, (_, n, _)) in enumerate(zip(ys, shapes)):
        arr[i] = lib.W4A4Sibling(qa[i].data_ptr(), sx_pairs[i].data_ptr(), weight_operand[i].data_ptr(),
                                 weight_scale_pairs[i].data_ptr(), mid[i].data_ptr(), l1cat[i].data_ptr(),
                                 mid[i].shape[2], _vp(bias[i]), n, y.data_ptr(), n)
    lib.call("svdq_w4a4_gemm_siblings", arr, count, operand, m, k, group_size, int(out_f32), _stream(dev))
    return ys


@w4a4_gemm_siblings.register_fake
def _(qa, sx_pairs, weight_operand, weight_scale_pairs, mid, l1cat, bias, group_size, operand, out_f32):
    return [a.new_empty((s.shape[1], w.shape[1]), dtype=torch.float32 if out_f32 else torch.bfloat16)
            for a, s, w in zip(qa, sx_pairs, weight_scale_pairs)]


@torch.library.custom_op("svdq::w4a16_gemm", mutates_args=())
def w4a16_gemm(xhat: Tensor, qweight: Tensor, weight_scales: Tensor, mid: Tensor, l1cat: Tensor,
               bias: Optional[Tensor], group_size: int, out_f32: bool, epi: int = 0, aux: Optional[Tensor] = None,
               vec: Optional[Tensor] = None) -> Tensor:
    """``y = xhat @ bf16(q * bf16(sw))^T + mid @ l1cat^T + bias`` (bf16 or float32 output), then the
    elementwise op ``epi`` as in ``w4a4_gemm``."""
    _need(xhat.is_cuda, RuntimeError, "svdq::w4a16_gemm needs GPU tensors")
    dev = xhat.device
    _check_dev("xhat", xhat, dev, torch.bfloat16)
    m, k = xhat.shape
    n = _check_gemm(qweight, weight_scales, mid, l1cat, bias, m, k, group_size, dev)
    _check_epi(epi, aux, vec, m, n, out_f32, dev)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev)
    lib.call("svdq_w4a16_gemm_epi", _vp(xhat), k, _vp(qweight), _vp(weight_scales), _vp(mid), _vp(l1cat),
             mid.shape[2], _vp(bias), m, n, k, group_size, _vp(y), n, int(out_f32), *_epi_args(epi, aux, vec, n),
             _stream(dev))
    return y


@w4a16_gemm.register_fake
def _(xhat, qweight, weight_scales, mid, l1cat, bias, group_size, out_f32, epi=0, aux=None, vec=None):
    return xhat.new_empty((xhat.shape[0], qweight.shape[0]), dtype=torch.float32 if out_f32 else torch.bfloat16)


@torch.library.custom_op("svdq::w4a16_gemm_siblings", mutates_args=())
def w4a16_gemm_siblings(xhat: list[Tensor], qweight: list[Tensor], weight_scales: list[Tensor], mid: list[Tensor],
                        l1cat: list[Tensor], bias: list[Optional[Tensor]], group_size: int,
                        out_f32: bool) -> list[Tensor]:
    """``w4a16_gemm`` of up to ``lib.SVDQ_MAX_SIBLINGS`` layers over the same rows (the i-th entry
    of every list belongs to layer i; each layer its own x_hat), in one launch when that pays
    (``svdq_w4a16_gemm_siblings``); each output is bit-identical to that layer's ``w4a16_gemm``."""
    count = len(xhat)
    _need(1 <= count <= lib.SVDQ_MAX_SIBLINGS, ValueError, f"1..{lib.SVDQ_MAX_SIBLINGS} layers, got {count}")
    _need(all(len(a) == count for a in (qweight, weight_scales, mid, l1cat, bias)), ValueError,
          "one entry per layer in every list")
    _need(xhat[0].is_cuda, RuntimeError, "svdq::w4a16_gemm_siblings needs GPU tensors")
    dev = xhat[0].device
    m, k = xhat[0].shape
    ns = []
    for i in range(count):
        _check_dev(f"layer {i}: xhat", xhat[i], dev, torch.bfloat16)
        _need(tuple(xhat[i].shape) == (m, k), ValueError,
              f"sibling layers need the same M and K, got {tuple(xhat[i].shape)} and {(m, k)}")
        ns.append(_check_gemm(qweight[i], weight_scales[i], mid[i], l1cat[i], bias[i], m, k, group_size, dev))
    ys = [torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=dev) for n in ns]
    arr = (lib.W4A16Sibling * count)()
    for i, (y, n) in enumerate(zip(ys, ns)):
        arr[i] = lib.W4A16Sibling(xhat[i].data_ptr(), k, qweight[i].data_ptr(), weight_scales[i].data_ptr(),
                                  mid[i].data_ptr(), l1cat[i].data_ptr(), mid[i].shape[2], _vp(bias[i]), n,
                                  y.data_ptr(), n)
    lib.call("svdq_w4a16_gemm_siblings", arr, count, m, k, group_size, int(out_f32), _stream(dev))
    return ys


@w4a16_gemm_siblings.register_fake
def _(xhat, qweight, weight_scales, mid, l1cat, bias, group_size, out_f32):
    return [x.new_empty((x.shape[0], w.shape[0]), dtype=torch.float32 if out_f32 else torch.bfloat16)
            for x, w in zip(xhat, qweight)]


# ---- stand-in block normalizations -------------------------------------------------------------
@torch.library.custom_op("svdq::gate_op", mutates_args=())
def gate_op(y: Tensor, aux: Tensor, op: int) -> Tensor:
    """``aux * sigmoid(y)`` (op ``EPILOGUES["mul_sigmoid"]``) or ``silu(aux) * y`` (op
    ``EPILOGUES["silu_mul"]``), elementwise over bf16 tensors of one shape, rounded as the torch ops
    on bf16 tensors; one pass (``svdq_gate_op``)."""
    _need(y.is_cuda, RuntimeError, "svdq::gate_op needs GPU tensors")
    _need(op in (EPILOGUES["mul_sigmoid"], EPILOGUES["silu_mul"]), ValueError, f"op={op}")
    _check_dev("y", y, y.device, torch.bfloat16)
    _check_dev("aux", aux, y.device, torch.bfloat16)
    _need(y.shape == aux.shape, ValueError, f"y {tuple(y.shape)} and aux {tuple(aux.shape)} differ")
    y2, a2 = y.contiguous(), aux.contiguous()
    y2 = y2 if y2.data_ptr() % 16 == 0 else y2.clone()
    a2 = a2 if a2.data_ptr() % 16 == 0 else a2.clone()
    out = torch.empty_like(y2)
    lib.call("svdq_gate_op", op, _vp(y2), _vp(a2), _vp(out), y2.numel(), _stream(y.device))
    return out


@gate_op.register_fake
def _(y, aux, op):
    return torch.empty_like(y)


@torch.library.custom_op("svdq::rms_norm_modulate", mutates_args=())
def rms_norm_modulate(x: Tensor, weight: Tensor, shift: Tensor, eps: float) -> Tensor:
    """``bf16(bf16(x * rsqrt(mean(x^2) + eps) * weight) + shift)`` over the last dimension of a
    bf16 ``x`` [..., H] (H % 8 == 0): the stand-in block's adaptive RMS norm (weight = 1 + scale)."""
    _need(x.is_cuda, RuntimeError, "svdq::rms_norm_modulate needs GPU tensors")
    dev = x.device
    h = x.shape[-1]
    for name, t in (("weight", weight), ("shift", shift)):
        _check_dev(name, t, dev, torch.bfloat16)
        _need(t.numel() == h, ValueError, f"{name} must have {h} elements, got {t.numel()}")
    _need(x.dtype == torch.bfloat16, TypeError, f"x must be bf16, got {x.dtype}")
    x2 = x.reshape(-1, h)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    y = torch.empty((x2.shape[0], h), dtype=torch.bfloat16, device=dev)
    lib.call("svdq_rms_norm_modulate", _vp(x2), x2.stride(0), _vp(weight), _vp(shift),
             x2.shape[0], h, ctypes.c_float(eps), _vp(y), h, _stream(dev))
    return y.view(x.shape)


@rms_norm_modulate.register_fake
def _(x, weight, shift, eps):
    return torch.empty_like(x)


def _rows16(t: Tensor, h: int) -> Tensor:
    """[..., h] as rows with unit stride, a leading dimension % 8 == 0 and a 16-byte aligned start."""
    t2 = t.reshape(-1, h)
    if t2.stride(-1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    if t2.data_ptr() % 16:
        t2 = t2.clone()
    return t2


@torch.library.custom_op("svdq::residual_rms_norm_modulate", mutates_args=())
def residual_rms_norm_modulate(x: Tensor, v: Tensor, gate: Tensor, weight: Tensor, shift: Tensor,
                               eps: float) -> tuple[Tensor, Tensor]:
    """``xo = torch.addcmul(x, gate, v)`` (bf16, one rounding) and ``rms_norm_modulate(xo, weight,
    shift, eps)`` in one pass; returns ``(xo, y)``.  ``x``, ``v`` bf16 [..., H] of one shape,
    ``gate``, ``weight``, ``shift`` bf16 [H]."""
    _need(x.is_cuda, RuntimeError, "svdq::residual_rms_norm_modulate needs GPU tensors")
    dev = x.device
    h = x.shape[-1]
    _need(x.dtype == torch.bfloat16 and v.dtype == torch.bfloat16, TypeError, "x and v must be bf16")
    _need(v.shape == x.shape and v.device == dev, ValueError, f"v {tuple(v.shape)} must match x {tuple(x.shape)}")
    for name, t in (("gate", gate), ("weight", weight), ("shift", shift)):
        _check_dev(name, t, dev, torch.bfloat16)
        _need(t.numel() == h, ValueError, f"{name} must have {h} elements, got {t.numel()}")
    gate, weight, shift = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (gate, weight, shift))
    x2, v2 = _rows16(x, h), _rows16(v, h)
    xo = torch.empty((x2.shape[0], h), dtype=torch.bfloat16, device=dev)
    y = torch.empty_like(xo)
    lib.call("svdq_residual_rms_norm_modulate", _vp(x2), x2.stride(0), _vp(v2), v2.stride(0), _vp(gate),
             _vp(weight), _vp(shift), x2.shape[0], h, ctypes.c_float(eps), _vp(xo), h, _vp(y), h, _stream(dev))
    return xo.view(x.shape), y.view(x.shape)


@residual_rms_norm_modulate.register_fake
def _(x, v, gate, weight, shift, eps):
    return torch.empty_like(x), torch.empty_like(x)


@torch.library.custom_op("svdq::head_rms_rope", mutates_args=())
def head_rms_rope(t: Tensor, cos: Tensor, sin: Tensor, eps: float) -> Tensor:
    """Per-head RMS norm of ``t`` [T, heads, 128] (bf16) followed by the rotate-half rotary
    embedding with the position tables ``cos`` / ``sin`` [T, >= 64] (bf16; columns 0..63 read)."""
    _need(t.is_cuda, RuntimeError, "svdq::head_rms_rope needs GPU tensors")
    dev = t.device
    _need(t.dim() == 3 and t.shape[-1] == 128, ValueError, f"t must be [T, heads, 128], got {tuple(t.shape)}")
    _need(t.dtype == torch.bfloat16, TypeError, f"t must be bf16, got {t.dtype}")
    tok, heads = t.shape[0], t.shape[1]
    for name, tab in (("cos", cos), ("sin", sin)):
        _check_dev(name, tab, dev, torch.bfloat16)
        _need(tab.dim() == 2 and tab.shape[0] == tok and tab.shape[1] >= 64 and tab.stride(-1) == 1, ValueError,
              f"{name} must be [{tok}, >= 64] with unit column stride, got {tuple(tab.shape)}")
    _need(cos.stride(0) == sin.stride(0), ValueError, "cos and sin must share a row stride")
    t = t.contiguous()
    out = torch.empty_like(t)
    lib.call("svdq_head_rms_rope", _vp(t), tok, heads, _vp(cos), _vp(sin), cos.stride(0), ctypes.c_float(eps),
             _vp(out), _stream(dev))
    return out


@head_rms_rope.register_fake
def _(t, cos, sin, eps):
    return torch.empty_like(t)


def _attention(q: Tensor, k: Tensor, v: Tensor, scale: float, cos: Optional[Tensor], sin: Optional[Tensor],
               eps: float) -> Tensor:
    _need(q.is_cuda, RuntimeError, "svdq::attention needs GPU tensors")
    dev = q.device
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need(t.device == dev, ValueError, f"{name} is on {t.device}, expected {dev}")
        _need(t.dtype == torch.bfloat16, TypeError, f"{name} must be torch.bfloat16, got {t.dtype}")
        _need(t.dim() == 3 and t.shape[-1] == 128, ValueError, f"{name} must be [T, heads, 128], got {tuple(t.shape)}")
    tok, heads, kvh = q.shape[0], q.shape[1], k.shape[1]
    _need(k.shape == v.shape and k.shape[0] == tok, ValueError,
          f"k and v must both be [{tok}, Hkv, 128], got {tuple(k.shape)} and {tuple(v.shape)}")
    _need(heads % kvh == 0, ValueError, f"query heads ({heads}) must be a multiple of key / value heads ({kvh})")
    _need(k.stride(0) == v.stride(0), ValueError, "k and v must share a row stride")

    def rows(t: Tensor) -> Tensor:   # unit stride inside a row of heads, 16-byte aligned rows
        ok = t.stride(2) == 1 and t.stride(1) == 128 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
        return t if ok else t.contiguous()
    q, k, v = rows(q), rows(k), rows(v)
    if k.stride(0) != v.stride(0):
        k, v = k.contiguous(), v.contiguous()
    out = torch.empty((tok, heads, 128), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(lib.load().svdq_attention_workspace(tok, heads), dtype=torch.uint8, device=dev)
    if cos is None:
        lib.call("svdq_attention_fwd", _vp(q), q.stride(0), _vp(k), _vp(v), k.stride(0), tok, heads, kvh,
                 ctypes.c_float(scale), _vp(out), out.stride(0), _vp(ws), _stream(dev))
        return out
    for name, t in (("cos", cos), ("sin", sin)):
        _need(t is not None and t.device == dev and t.dtype == torch.bfloat16, TypeError,
              f"{name} must be a bf16 tensor on {dev}")
        _need(t.dim() == 2 and t.shape[0] >= tok and t.shape[1] >= 64, ValueError,
              f"{name} must be [T, >= 64], got {tuple(t.shape)}")
    cos, sin = (t if t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0 else t.contiguous()
                for t in (cos, sin))
    if cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    lib.call("svdq_attention_fwd_qnorm", _vp(q), q.stride(0), _vp(k), _vp(v), k.stride(0), tok, heads, kvh,
             ctypes.c_float(scale), _vp(cos), _vp(sin), cos.stride(0), ctypes.c_float(eps), _vp(out), out.stride(0),
             _vp(ws), _stream(dev))
    return out


@torch.library.custom_op("svdq::attention", mutates_args=())
def attention(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    """Softmax attention ``softmax(scale q k^T) v`` without a mask: ``q`` [T, H, 128], ``k`` / ``v``
    [T, Hkv, 128] (bf16, H a multiple of Hkv: query head h reads key / value head h // (H // Hkv))
    -> [T, H, 128] bf16.  Rows may be strided (last two dimensions contiguous)."""
    return _attention(q, k, v, scale, None, None, 0.0)


@torch.library.custom_op("svdq::attention_qnorm", mutates_args=())
def attention_qnorm(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor, eps: float, scale: float) -> Tensor:
    """``attention(head_rms_rope(q, cos, sin, eps), k, v, scale)`` with the per-head norm and rotary
    embedding of q applied as the kernel loads q (no normalized copy of q; a normalized value may
    differ by one bf16 ulp where the mean of squares sits at a rounding boundary)."""
    return _attention(q, k, v, scale, cos, sin, eps)


@attention_qnorm.register_fake
def _(q, k, v, cos, sin, eps, scale):
    return q.new_empty((q.shape[0], q.shape[1], 128))


@attention.register_fake
def _(q, k, v, scale):
    return q.new_empty((q.shape[0], q.shape[1], 128))
