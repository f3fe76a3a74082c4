"""``SVDQuantLinear`` / ``SVDQuantLoRAAdapter``: the drop-in module boundary.

Mirror of reference ``src/krea2_svdquant/runtime/linear.py``: same constructor
``SVDQuantLinear(state, backend)``, same buffers (``smooth_scale``, ``qweight``,
``weight_scales``, ``l1``, ``l2``, ``bias``; persistent, so ``.to()`` and state dicts move
them), same ``add_lora_adapter(down, up, *, scale, network_alpha)`` validation and
``state`` property, ``_forward_base`` (the quantized linear alone) and ``forward``
(``_forward_base`` plus every adapter).

Differences, both deliberate:

* the backends are this package's gfx950 kernels; ``auto`` resolves to ``hip_gfx950`` on a
  gfx950 device and the reference's simulation / Triton / Gluon backends raise instead of
  being emulated -- there is no silent fallback (reference ``linear.py:133-153`` swallows
  kernel errors into the simulation);
* LoRA adapters are fused into the two kernels (down projection in the activation pass,
  up projection in the GEMM epilogue) instead of running as extra GEMMs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from ..config import BackendKind
from ..quant.state import SVDQuantLinearState
from ..kernels.hip.backend import PreparedLayer, forward_prepared, prepare_layer

_HIP_MODES = {BackendKind.HIP_GFX950: "w4a4", BackendKind.HIP_GFX950_W4A16: "w4a16"}


class SVDQuantLoRAAdapter(nn.Module):
    """Inference-only LoRA branch attached to a quantized linear (reference ``linear.py:11-45``).

    ``multiplier = scale * network_alpha / rank`` with ``network_alpha`` defaulting to the rank.
    ``forward`` evaluates the branch on its own (``up(down(x)) * multiplier``); inside
    ``SVDQuantLinear`` the branch runs fused in the gfx950 kernels instead.
    """

    def __init__(self, down_weight: torch.Tensor, up_weight: torch.Tensor, *, scale: float = 1.0,
                 network_alpha: float | None = None) -> None:
        super().__init__()
        if down_weight.ndim != 2 or up_weight.ndim != 2:
            raise ValueError("LoRA down/up weights must be rank-2 tensors")
        rank = int(down_weight.shape[0])
        if rank <= 0:
            raise ValueError("LoRA rank must be positive")
        if int(up_weight.shape[1]) != rank:
            raise ValueError(f"LoRA shape mismatch: down={tuple(down_weight.shape)} up={tuple(up_weight.shape)}")
        self.rank = rank
        self.scale = float(scale)
        self.network_alpha = float(network_alpha) if network_alpha is not None else float(rank)
        self.register_buffer("down_weight", down_weight.contiguous(), persistent=True)
        self.register_buffer("up_weight", up_weight.contiguous(), persistent=True)

    @property
    def multiplier(self) -> float:
        return self.scale * (self.network_alpha / self.rank)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        down = self.down_weight.to(dtype=x.dtype)
        up = self.up_weight.to(dtype=x.dtype)
        return F.linear(F.linear(x, down), up) * self.multiplier


def is_gfx950(device: torch.device | None = None) -> bool:
    if not torch.cuda.is_available():
        return False
    props = torch.cuda.get_device_properties(device or torch.cuda.current_device())
    return getattr(props, "gcnArchName", "").split(":")[0] == "gfx950"


class SVDQuantLinear(nn.Module):
    """Quantized linear layer with the gfx950 kernels as its backend."""

    def __init__(self, state: SVDQuantLinearState, backend: BackendKind | str = BackendKind.AUTO):
        super().__init__()
        self.backend = BackendKind(backend)
        self.group_size = int(state.group_size)
        self.original_shape = tuple(int(v) for v in state.original_shape)
        self.qweight_packed = bool(state.qweight_packed)
        self.padded_in_features = state.padded_in_features
        self.register_buffer("smooth_scale", state.smooth_scale.contiguous(), persistent=True)
        self.register_buffer("qweight", state.qweight.contiguous(), persistent=True)
        self.register_buffer("weight_scales", state.weight_scales.contiguous(), persistent=True)
        self.register_buffer("l1", state.l1.contiguous(), persistent=True)
        self.register_buffer("l2", state.l2.contiguous(), persistent=True)
        if state.bias is None:
            self.bias = None
        else:
            self.register_buffer("bias", state.bias.contiguous(), persistent=True)
        self.lora_adapters = nn.ModuleList()
        self._prepared: dict[bool, tuple[tuple, PreparedLayer]] = {}

    # -- reference API -------------------------------------------------------------------
    def add_lora_adapter(self, down_weight: torch.Tensor, up_weight: torch.Tensor, *, scale: float = 1.0,
                         network_alpha: float | None = None) -> None:
        """Attach an inference LoRA adapter (reference ``linear.py:88-111``)."""
        expected_out, expected_in = self.original_shape
        if tuple(down_weight.shape[1:]) != (expected_in,):
            raise ValueError(f"LoRA down input mismatch for SVDQuantLinear: expected {expected_in}, "
                             f"got {tuple(down_weight.shape)}")
        if int(up_weight.shape[0]) != expected_out:
            raise ValueError(f"LoRA up output mismatch for SVDQuantLinear: expected {expected_out}, "
                             f"got {tuple(up_weight.shape)}")
        self.lora_adapters.append(SVDQuantLoRAAdapter(down_weight, up_weight, scale=scale,
                                                      network_alpha=network_alpha))
        self._prepared.clear()

    @property
    def state(self) -> SVDQuantLinearState:
        return SVDQuantLinearState(
            smooth_scale=self.smooth_scale, qweight=self.qweight, weight_scales=self.weight_scales,
            l1=self.l1, l2=self.l2, bias=self.bias, group_size=self.group_size,
            original_shape=self.original_shape, qweight_packed=self.qweight_packed,
            padded_in_features=self.padded_in_features)

    def _forward_base(self, x: torch.Tensor) -> torch.Tensor:
        """The quantized linear without LoRA adapters."""
        return forward_prepared(x, self._prepare(x.device, with_adapters=False), mode=self._mode(x.device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.lora_adapters:
            return self._forward_base(x)
        return forward_prepared(x, self._prepare(x.device, with_adapters=True), mode=self._mode(x.device))

    def forward_epilogue(self, x: torch.Tensor, epilogue: str, aux: torch.Tensor,
                         vec: torch.Tensor | None = None) -> torch.Tensor:
        """``forward(x)`` followed by an elementwise op fused into the kernel's store (o = the
        layer output): ``"mul_sigmoid"`` -> ``aux * sigmoid(o)``, ``"silu_mul"`` ->
        ``silu(aux) * o``, ``"residual_gate"`` -> ``aux + vec * o``, each op rounded to bf16 as
        the same torch ops on bf16 tensors are.  Not in the reference module (its blocks run
        these ops in diffusers); the stand-in Krea-2 block uses it for SwiGLU, the attention
        output gate and the gated residuals."""
        prep = self._prepare(x.device, with_adapters=bool(self.lora_adapters))
        return forward_prepared(x, prep, mode=self._mode(x.device), epilogue=epilogue, aux=aux, vec=vec)

    # -- backend plumbing ----------------------------------------------------------------
    def resolved_backend(self, device: torch.device | None = None) -> BackendKind:
        if self.backend is BackendKind.AUTO:
            if not is_gfx950(device):
                raise RuntimeError("backend 'auto' needs a gfx950 (MI355X) device for the HIP backend")
            return BackendKind.HIP_GFX950
        if self.backend not in _HIP_MODES:
            raise NotImplementedError(
                f"backend {self.backend.value!r} is not part of this package; available: "
                f"{', '.join(b.value for b in _HIP_MODES)} (and 'auto')")
        return self.backend

    def _mode(self, device: torch.device) -> str:
        return _HIP_MODES[self.resolved_backend(device)]

    def _buffers_key(self, device: torch.device) -> tuple:
        # storage and version counter of every buffer: in-place edits bump the version
        bufs = (self.qweight, self.smooth_scale, self.weight_scales, self.l1, self.l2, self.bias)
        return (str(device),) + tuple((b.data_ptr(), b._version) if b is not None else None for b in bufs)

    def _adapters_key(self) -> tuple:
        # each adapter's identity, multiplier (read on every forward, as the reference does) and
        # weights (storage and version)
        return tuple((id(a), a.multiplier, a.down_weight.data_ptr(), a.down_weight._version, a.up_weight.data_ptr(),
                      a.up_weight._version) for a in self.lora_adapters)

    def _prepare(self, device: torch.device, with_adapters: bool) -> PreparedLayer:
        """The kernels' operands of this layer, cached per (buffers, adapters).  The adapter entry
        shares the base entry's weight operands (prepare_layer's ``base``)."""
        self.resolved_backend(device)
        base_key = self._buffers_key(device)
        hit = self._prepared.get(False)
        if hit is None or hit[0] != base_key:
            self._prepared.clear()
            hit = (base_key, prepare_layer(self.state, (), device))
            self._prepared[False] = hit
        if not with_adapters:
            return hit[1]
        key = base_key + self._adapters_key()
        ahit = self._prepared.get(True)
        if ahit is None or ahit[0] != key:
            ahit = (key, prepare_layer(self.state, list(self.lora_adapters), device, base=hit[1]))
            self._prepared[True] = ahit
        return ahit[1]

    def invalidate_prepared(self) -> None:
        """Drop the cached per-layer kernel operands (call after editing buffers in place)."""
        self._prepared.clear()

    def _apply(self, fn, *args, **kwargs):
        self._prepared.clear()
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self._prepared.clear()
        return super()._load_from_state_dict(*args, **kwargs)
