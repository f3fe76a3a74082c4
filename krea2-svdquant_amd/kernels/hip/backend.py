"""The gfx950 backend function: ``fn(x, state) -> y`` like reference
``kernels/triton/generic_int4.py:227-244`` (``svdquant_linear_triton_generic``).

Two launches per layer forward:

* W4A4  (``mode="w4a4"``):  ``svdq::act_quant`` (codes, scales, mid) -> ``svdq::w4a4_gemm``;
* W4A16 (``mode="w4a16"``): ``svdq::act_quant`` (x_hat, mid)         -> ``svdq::w4a16_gemm``.

LoRA adapters (reference ``runtime/linear.py:11-45``) are fused: their down projections run
in the activation pass on the raw x (times each adapter's multiplier) and their up
projections are concatenated behind ``l1`` in the GEMM epilogue.  Per-layer constants
(``1/s``, the concatenated ``l1 | up`` matrix, the padded ``l2``) are built once by
``prepare_layer`` and cached by ``SVDQuantLinear``.

Errors follow the reference: ``ValueError`` for shapes, ``TypeError`` for dtypes,
``RuntimeError`` for an unusable backend (no GPU, unpacked checkpoint, missing library).
Nothing falls back to another implementation.
"""
from __future__ import annotations

import math

import weakref
from dataclasses import dataclass
from typing import Optional, Sequence

import torch
from torch import Tensor

from ...quant.state import SVDQuantLinearState
from . import ops


FAST_GROUPS = (64, 128)
"""Group sizes with the tuned kernels; any other multiple of 16 dividing K takes the generic
kernels (int8 operands, K in steps of 16, a rescale at every group boundary)."""


@dataclass
class PreparedLayer:
    """Device-resident per-layer operands of the two kernels."""
    srs: Tensor                  # f32 [2Kp]: s, RN(1/s)
    l2: Tensor                   # bf16 [r, Kp]
    l1cat: Tensor                # bf16 [N, RTp] = [l1 | up_1 | ... | 0]
    lora_down: Optional[Tensor]  # bf16 [rl, Kp]
    lora_mult: Optional[Tensor]  # f32 [rl]
    qweight: Tensor              # uint8 [N, Kp/2]
    weight_scales: Tensor        # fp16 [N, Kp/G]
    scale_pairs: dict            # operand code -> int32 [Kp/G, N] W4A4 scale-MFMA operand (lazy)
    operands: dict               # operand code -> W4A4 weight operand (uint8 [N, Kp], e3m2 planar) (lazy)
    bias: Optional[Tensor]       # bf16 [N]
    group_size: int
    n: int
    k: int                       # logical in_features
    kp: int                      # padded in_features
    rtp: int

    @property
    def device(self) -> torch.device:
        return self.qweight.device

    def weight_operand(self, operand: int) -> Tensor:
        codes = self.operands.get(operand)
        if codes is None:
            codes = self.operands[operand] = ops.prepare_weight_operand(self.qweight, operand)
        return codes

    def weight_scale_pairs(self, operand: int) -> Tensor:
        pairs = self.scale_pairs.get(operand)
        if pairs is None:
            pairs = self.scale_pairs[operand] = ops.prepare_weight_scales(self.weight_scales, operand)
        return pairs


def _pad_cols(t: Tensor, kp: int, value: float = 0.0) -> Tensor:
    if t.shape[-1] == kp:
        return t.contiguous()
    out = t.new_full((*t.shape[:-1], kp), value)
    out[..., : t.shape[-1]] = t
    return out


def prepare_layer(state: SVDQuantLinearState, adapters: Sequence = (),
                  device: torch.device | str | None = None, *, base: Optional[PreparedLayer] = None) -> PreparedLayer:
    """Validate a packed state and build the kernels' per-layer operands on ``device``.

    ``adapters`` are objects with ``down_weight`` [rl, K], ``up_weight`` [N, rl] and
    ``multiplier`` (``SVDQuantLoRAAdapter``).  ``base``: the same layer prepared without
    adapters; its smoothing constants, weight buffers and (lazily built) weight operands are
    shared instead of rebuilt, so a layer holds one expanded weight operand however many adapter
    sets it is prepared with.
    """
    if not state.qweight_packed:
        raise RuntimeError("HIP gfx950 backend expects packed uint8 qweight (qweight_packed=True)")
    dev = torch.device(device) if device is not None else state.qweight.device
    if dev.type != "cuda":
        raise RuntimeError("HIP gfx950 backend needs its state on a GPU device")
    n, k = (int(v) for v in state.original_shape)
    qweight = state.qweight.to(dev).contiguous()
    if qweight.dtype != torch.uint8 or qweight.dim() != 2 or qweight.shape[0] != n:
        raise TypeError(f"qweight must be uint8 [{n}, Kp/2], got {qweight.dtype} {tuple(qweight.shape)}")
    kp = int(state.padded_in_features or qweight.shape[1] * 2)
    if kp != qweight.shape[1] * 2 or kp < k:
        raise ValueError(f"padded_in_features={kp} inconsistent with qweight {tuple(qweight.shape)} and K={k}")
    g = int(state.group_size)
    if kp % g:
        raise ValueError(f"padded K={kp} is not a multiple of group_size={g}")
    scales = state.weight_scales.to(dev)
    if scales.dtype != torch.float16:
        raise TypeError(f"weight_scales must be float16 (checkpoint layout), got {scales.dtype}")
    if tuple(scales.shape) != (n, kp // g):
        raise ValueError(f"weight_scales must be [{n}, {kp // g}], got {tuple(scales.shape)}")
    if g not in FAST_GROUPS and kp % 64:
        # The generic-group kernels step K by 64 columns; the reference pads K only to a multiple of
        # the group (quant/pack.py:12-16).  Pad further, to a multiple of lcm(group, 64): zero
        # activation columns (smoothing 1), weight codes 0 (nibble 8) with scale 1, zero low-rank
        # and LoRA down columns.  The added groups' products are exactly zero, so every output is
        # the unpadded layer's.
        kq = -(-kp // math.lcm(g, 64)) * math.lcm(g, 64)
        qweight = _pad_cols(qweight, kq // 2, 0x88)
        scales = _pad_cols(scales, kq // g, 1.0)
        kp = kq
    smooth = _pad_cols(state.smooth_scale.to(dev, torch.bfloat16), kp, 1.0)
    l1 = state.l1.to(dev, torch.bfloat16)
    l2 = _pad_cols(state.l2.to(dev, torch.bfloat16), kp)
    r = int(l2.shape[0])
    if tuple(l1.shape) != (n, r):
        raise ValueError(f"l1 must be [{n}, {r}], got {tuple(l1.shape)}")
    downs, ups, mults = [], [], []
    for ad in adapters:
        down = ad.down_weight.to(dev, torch.bfloat16)
        up = ad.up_weight.to(dev, torch.bfloat16)
        downs.append(_pad_cols(down, kp))
        ups.append(up)
        mults.append(torch.full((down.shape[0],), float(ad.multiplier), dtype=torch.float32, device=dev))
    rl = sum(d.shape[0] for d in downs)
    rtp = ops.rank_padded(r + rl)
    l1cat = torch.zeros((n, rtp), dtype=torch.bfloat16, device=dev)
    l1cat[:, :r] = l1
    col = r
    for up in ups:
        l1cat[:, col: col + up.shape[1]] = up
        col += up.shape[1]
    bias = None if state.bias is None else state.bias.to(dev, torch.bfloat16).contiguous()
    shared = base is not None and base.device == dev and base.kp == kp and base.n == n
    return PreparedLayer(
        srs=base.srs if shared else ops.prepare_smooth(smooth.contiguous()),
        l2=l2.contiguous(),
        l1cat=l1cat,
        lora_down=torch.cat(downs, 0).contiguous() if downs else None,
        lora_mult=torch.cat(mults, 0).contiguous() if mults else None,
        qweight=base.qweight if shared else qweight,
        weight_scales=base.weight_scales if shared else scales.contiguous(),
        scale_pairs=base.scale_pairs if shared else {},
        operands=base.operands if shared else {},
        bias=bias,
        group_size=g, n=n, k=k, kp=kp, rtp=rtp,
    )


def _flatten(x: Tensor) -> tuple[Tensor, tuple[int, ...]]:
    if x.ndim < 2:
        raise ValueError(f"expected [..., K] activation, got shape {tuple(x.shape)}")
    return x.reshape(-1, x.shape[-1]).contiguous(), tuple(x.shape[:-1])


def _aligned(t: Tensor) -> Tensor:
    """``t`` itself when its storage starts on 16 bytes (the kernels' vector loads), else a copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _epilogue_operands(epilogue: str, aux: Optional[Tensor], vec: Optional[Tensor], m: int, n: int,
                       device: torch.device) -> tuple[int, Optional[Tensor], Optional[Tensor]]:
    if epilogue not in ops.EPILOGUES:
        raise ValueError(f"epilogue must be one of {sorted(ops.EPILOGUES)}, got {epilogue!r}")
    epi = ops.EPILOGUES[epilogue]
    if epi == 0:
        if aux is not None or vec is not None:
            raise ValueError("aux / vec given without an epilogue op")
        return epi, None, None
    if aux is None or aux.shape[-1] != n or aux.numel() != m * n:
        raise ValueError(f"epilogue {epilogue!r} needs aux of shape [..., {n}] with {m} rows")
    if aux.device != device or aux.dtype != torch.bfloat16:
        raise TypeError(f"aux must be bfloat16 on {device}, got {aux.dtype} on {aux.device}")
    aux2 = _aligned(aux.reshape(m, n).contiguous())
    vec2 = None
    if epi == ops.EPILOGUES["residual_gate"]:
        if vec is None or vec.numel() != n:
            raise ValueError(f"epilogue 'residual_gate' needs vec with {n} entries")
        vec2 = _aligned(vec.to(device, torch.bfloat16).reshape(n).contiguous())
    elif vec is not None:
        raise ValueError("vec is only used by epilogue 'residual_gate'")
    return epi, aux2, vec2


def forward_prepared(x: Tensor, prep: PreparedLayer, *, mode: str = "w4a4", out_f32: bool = False,
                     exact_div: bool = False, operand: str = "e3m2", epilogue: str = "none",
                     aux: Optional[Tensor] = None, vec: Optional[Tensor] = None) -> Tensor:
    """One SVDQuantLinear forward on prepared operands; returns [..., N].

    ``operand`` picks the W4A4 MFMA: ``"e3m2"`` (FP6 MFMA, default: twice the FP8 rate),
    ``"e4m3"`` (FP8 MFMA) or ``"i8"`` (INT8 MFMA); all compute the same exact integer group sums.
    Layers whose group size is not 64 or 128 always take the generic int8 kernels.
    ``epilogue`` fuses an elementwise op into the GEMM's bf16 store (o = the layer output, bf16
    rounding after every op as with the unfused torch ops): ``"mul_sigmoid"`` gives
    ``aux * sigmoid(o)``, ``"silu_mul"`` gives ``silu(aux) * o`` and ``"residual_gate"`` gives
    ``aux + vec * o``; ``aux`` has the output's shape, ``vec`` is [N].
    """
    if not x.is_cuda:
        raise RuntimeError("HIP gfx950 backend needs a GPU tensor")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"HIP gfx950 backend takes bfloat16 activations, got {x.dtype}")
    if x.device != prep.device:
        raise ValueError(f"activation on {x.device}, layer on {prep.device}")
    x2, lead = _flatten(x)
    k = x2.shape[1]
    if k > prep.kp:
        raise ValueError(f"activation K={k} exceeds packed weight K={prep.kp}")
    if k != prep.kp:
        x2 = _pad_cols(x2, prep.kp)
    epi, aux2, vec2 = _epilogue_operands(epilogue, aux, vec, x2.shape[0], prep.n, x.device)
    if mode == "w4a4":
        if operand not in ops.OPERAND_NAMES:
            raise ValueError(f"operand must be 'e4m3', 'e3m2' or 'i8', got {operand!r}")
        opc = ops.OPERAND_NAMES[operand]
        generic = prep.group_size not in FAST_GROUPS
        if generic:
            # group sizes other than 64 / 128: the generic kernels, int8 operands quantized from x_hat
            opc = ops.OPERAND_I8
        qa, sx, _, _, mid = ops.act_quant(x2, prep.srs, prep.l2, prep.lora_down, prep.lora_mult,
                                          prep.group_size, prep.rtp, opc, False, generic, exact_div, True)
        y = ops.w4a4_gemm(qa, sx, prep.weight_operand(opc), prep.weight_scale_pairs(opc), mid, prep.l1cat,
                          prep.bias, prep.group_size, opc, out_f32, epi, aux2, vec2)
    elif mode == "w4a16":
        _, _, _, xhat, mid = ops.act_quant(x2, prep.srs, prep.l2, prep.lora_down, prep.lora_mult,
                                           prep.group_size, prep.rtp, ops.OPERAND_NONE, False, True,
                                           exact_div)
        y = ops.w4a16_gemm(xhat, prep.qweight, prep.weight_scales, mid, prep.l1cat, prep.bias,
                           prep.group_size, out_f32, epi, aux2, vec2)
    else:
        raise ValueError(f"mode must be 'w4a4' or 'w4a16', got {mode!r}")
    return y.reshape(*lead, prep.n)


def forward_prepared_siblings(x: Tensor, preps: Sequence[PreparedLayer], *, mode: str = "w4a4",
                              out_f32: bool = False, exact_div: bool = False, operand: str = "e3m2") -> list[Tensor]:
    """Forwards of sibling layers (same input ``x``, same K and group size) on prepared operands.
    W4A4: an activation pass per layer (each layer has its own smoothing; one launch for all when
    none has LoRA adapters, ``svdq::act_quant_siblings``), then the layers' GEMMs as one launch
    (``svdq::w4a4_gemm_siblings``).  W4A16: each layer's x_hat pass, then the layers' GEMMs as one
    launch where that pays (``svdq::w4a16_gemm_siblings``).  Every output is bit-identical to
    ``forward_prepared(x, prep, mode=mode)`` of its layer."""
    if not x.is_cuda:
        raise RuntimeError("HIP gfx950 backend needs a GPU tensor")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"HIP gfx950 backend takes bfloat16 activations, got {x.dtype}")
    if not 1 <= len(preps) <= ops.lib.SVDQ_MAX_SIBLINGS:
        raise ValueError(f"1..{ops.lib.SVDQ_MAX_SIBLINGS} sibling layers, got {len(preps)}")
    p0 = preps[0]
    for p in preps:
        if p.device != x.device:
            raise ValueError(f"activation on {x.device}, layer on {p.device}")
        if (p.kp, p.group_size) != (p0.kp, p0.group_size):
            raise ValueError("sibling layers need the same padded in_features and group size")
    if p0.group_size not in FAST_GROUPS:
        raise ValueError(f"sibling launch needs group size 64 or 128, got {p0.group_size}")
    if mode not in ("w4a4", "w4a16"):
        raise ValueError(f"mode must be 'w4a4' or 'w4a16', got {mode!r}")
    if operand not in ops.OPERAND_NAMES:
        raise ValueError(f"operand must be 'e4m3', 'e3m2' or 'i8', got {operand!r}")
    opc = ops.OPERAND_NAMES[operand]
    x2, lead = _flatten(x)
    if x2.shape[1] > p0.kp:
        raise ValueError(f"activation K={x2.shape[1]} exceeds packed weight K={p0.kp}")
    if x2.shape[1] != p0.kp:
        x2 = _pad_cols(x2, p0.kp)
    if mode == "w4a16":
        acts = [ops.act_quant(x2, p.srs, p.l2, p.lora_down, p.lora_mult, p.group_size, p.rtp, ops.OPERAND_NONE,
                              False, True, exact_div) for p in preps]
        ys = ops.w4a16_gemm_siblings([a[3] for a in acts], [p.qweight for p in preps],
                                     [p.weight_scales for p in preps], [a[4] for a in acts],
                                     [p.l1cat for p in preps], [p.bias for p in preps], p0.group_size, out_f32)
        return [y.reshape(*lead, p.n) for y, p in zip(ys, preps)]
    if opc == ops.OPERAND_E3M2 and all(p.lora_down is None and p.rtp == p0.rtp for p in preps):
        # one activation-pass launch for the layers (each its own smoothing) and one finalize
        flat = ops.act_quant_siblings(x2, [p.srs for p in preps], [p.l2 for p in preps], p0.group_size, p0.rtp,
                                      exact_div)
        acts = [(flat[3 * i], flat[3 * i + 1], None, None, flat[3 * i + 2]) for i in range(len(preps))]
    else:
        acts = [ops.act_quant(x2, p.srs, p.l2, p.lora_down, p.lora_mult, p.group_size, p.rtp, opc, False, False,
                              exact_div, True) for p in preps]
    ys = ops.w4a4_gemm_siblings([a[0] for a in acts], [a[1] for a in acts], [p.weight_operand(opc) for p in preps],
                                [p.weight_scale_pairs(opc) for p in preps], [a[4] for a in acts],
                                [p.l1cat for p in preps], [p.bias for p in preps], p0.group_size, opc, out_f32)
    return [y.reshape(*lead, p.n) for y, p in zip(ys, preps)]


# Prepared operands of the stateless entry, per state object: id(state) -> (key, PreparedLayer).  An
# entry is dropped when its state is garbage-collected and replaced when any buffer of the state
# or of an adapter is swapped or edited in place (storage and version counter in the key) or an
# adapter's multiplier changes.
_SEAM_CACHE: dict[int, tuple[tuple, PreparedLayer]] = {}


def _seam_key(state: SVDQuantLinearState, adapters: Sequence, device: torch.device) -> tuple:
    bufs = (state.qweight, state.smooth_scale, state.weight_scales, state.l1, state.l2, state.bias)
    return ((str(device), state.group_size)
            + tuple((b.data_ptr(), b._version) if b is not None else None for b in bufs)
            + tuple((id(a), a.multiplier, a.down_weight.data_ptr(), a.down_weight._version,
                     a.up_weight.data_ptr(), a.up_weight._version) for a in adapters))


def svdquant_linear_hip_gfx950(x: Tensor, state: SVDQuantLinearState, *, adapters: Sequence = (),
                               mode: str = "w4a4", out_f32: bool = False, operand: str = "e3m2") -> Tensor:
    """Stateless backend entry, the reference's backend-function seam
    (``kernels/triton/generic_int4.py:227``: ``fn(x, state)``).  The layer's kernel operands
    (including the expanded weight operand) are prepared on the first call for a state and kept
    while the state lives and its buffers are unchanged."""
    key = _seam_key(state, adapters, x.device)
    hit = _SEAM_CACHE.get(id(state))
    if hit is None or hit[0] != key:
        if hit is None:
            weakref.finalize(state, _SEAM_CACHE.pop, id(state), None)
        hit = (key, prepare_layer(state, adapters, x.device))
        _SEAM_CACHE[id(state)] = hit
    return forward_prepared(x, hit[1], mode=mode, out_f32=out_f32, operand=operand)


def svdquant_linear_hip_gfx950_w4a16(x: Tensor, state: SVDQuantLinearState, *, adapters: Sequence = (),
                                     out_f32: bool = False) -> Tensor:
    return svdquant_linear_hip_gfx950(x, state, adapters=adapters, mode="w4a16", out_f32=out_f32)
