"""Stand-in Krea-2 denoiser: whole denoise steps over the quantized linears of this package.

The reference wraps diffusers' ``Krea2Transformer2DModel`` (``src/krea2_svdquant/transformer.py:46-59``),
which is not installed here and whose block internals the reference does not contain.  This
module builds a transformer with the public dimensions the reference states (``README.md:27-37``:
28 blocks, hidden 6144, 48 query heads and 12 KV heads of 128, MLP 16384) and the eight
quantized linears per block under the reference's module names (``README.md:41-51``:
``transformer_blocks.{i}.attn.to_q`` ... ``transformer_blocks.{i}.ff.down``), so the checkpoint
reader and the module replacement address them as they would in the real model.

What the block computes around those linears is this module's own choice (single stream over
the concatenated text and latent tokens, modulation vectors fixed per block):

    h = rms_norm(x) * (1 + scale_a) + shift_a
    q, k, v = to_q(h), to_k(h), to_v(h);  per-head RMS norm of q and k;  rotary embedding on q, k
    a = softmax(q k^T / sqrt(d)) v  (48 query heads over 12 KV heads)
    x = x + gate_a * to_out.0(a * sigmoid(to_gate(h)))
    h = rms_norm(x) * (1 + scale_f) + shift_f
    x = x + gate_f * ff.down(silu(ff.gate(h)) * ff.up(h))

(the modulation's ``1 + scale`` runs as the norm's weight, the gated residuals as ``addcmul``
and the rotary embedding half by half: one bf16 rounding per fused op, fewer passes over x).
A denoise step is the 28 blocks over [text | latent] tokens followed by the Euler update of the
latent tokens, ``latent += dt * velocity``.  On the GPU every quantized linear runs on the gfx950
kernels (``SVDQuantLinear``), and so do the adaptive RMS norms and the per-head norm + rotary
embedding (``svdq::rms_norm_modulate``, ``svdq::head_rms_rope``: one pass each; ``NORMS = "torch"``
selects the torch ops) and the attention (``svdq::attention``, a flash-attention forward;
``ATTENTION = "sdpa"`` selects PyTorch's fused SDPA kernels), and so do the sigmoid gate and the
SwiGLU product (``svdq::gate_op``, one pass each, torch's bf16 rounding; ``GATES = "torch"`` selects
the torch ops); the gated residual adds run as ``torch.addcmul`` (on the CPU everything is torch).  With
``fused=True`` the sigmoid gate, the SwiGLU product and the two gated residual adds run inside
the stores of to_gate, ff.up, to_out.0 and ff.down instead.  The linears that read the same input
(to_q, to_k, to_v, to_gate; ff.gate, ff.up) run their GEMMs as one launch by default
(``run_grouped``; bit-identical to calling them one after another).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from functools import partial
from typing import Callable, Optional

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from ..kernels.hip import ops as hip_ops
from ..quant.state import SVDQuantLinearState
from .linear import SVDQuantLinear
from .siblings import run_concurrent, run_grouped

LINEAR_NAMES = ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_gate", "attn.to_out.0",
                "ff.gate", "ff.up", "ff.down")


@dataclass(frozen=True)
class Krea2Dims:
    """Public dimensions of Krea-2-Turbo's denoiser (reference ``README.md:27-37``)."""
    layers: int = 28
    hidden: int = 6144
    heads: int = 48
    kv_heads: int = 12
    head_dim: int = 128
    mlp: int = 16384

    def linear_shapes(self) -> dict[str, tuple[int, int]]:
        """(out_features, in_features) of each quantized linear of a block."""
        h, kv = self.hidden, self.kv_heads * self.head_dim
        return {"attn.to_q": (self.heads * self.head_dim, h), "attn.to_k": (kv, h), "attn.to_v": (kv, h),
                "attn.to_gate": (h, h), "attn.to_out.0": (h, self.heads * self.head_dim),
                "ff.gate": (self.mlp, h), "ff.up": (self.mlp, h), "ff.down": (h, self.mlp)}


def random_quantized_state(n: int, k: int, *, rank: int = 32, group_size: int = 64,
                           device: torch.device | str = "cuda", generator: torch.Generator | None = None
                           ) -> SVDQuantLinearState:
    """A random-init layer in the checkpoint layout, drawn directly in quantized form.

    Codes are uniform over the 16 INT4 values, fp16 group scales sit where a N(0, 0.02) weight's
    would (amax / 7 of a 64-sample group), the smoothing scale is uniform in [1, 4] and the
    factors are small Gaussians.  The kernels' work does not depend on the values, so this
    stands in for converting 224 dense random layers when only time is measured.
    """
    dev = torch.device(device)
    g = generator

    def randn(*shape):
        return torch.randn(*shape, device=dev, generator=g)

    kp = (k + group_size - 1) // group_size * group_size
    qweight = torch.randint(0, 256, (n, kp // 2), device=dev, generator=g, dtype=torch.uint8)
    scales = (0.02 * 2.5 / 7.0) * (0.8 + 0.4 * torch.rand(n, kp // group_size, device=dev, generator=g))
    smooth = 1.0 + 3.0 * torch.rand(k, device=dev, generator=g)
    return SVDQuantLinearState(
        smooth_scale=smooth.to(torch.bfloat16), qweight=qweight, weight_scales=scales.to(torch.float16),
        l1=(randn(n, rank) * 0.05).to(torch.bfloat16), l2=(randn(rank, k) / math.sqrt(k)).to(torch.bfloat16),
        bias=None, group_size=group_size, original_shape=(n, k), qweight_packed=True, padded_in_features=kp)


def rms_norm(x: Tensor, eps: float = 1e-6, weight: Optional[Tensor] = None) -> Tensor:
    """RMS norm over the last dimension, in x's dtype with an fp32 reduction; ``weight`` (the
    modulation's ``1 + scale``) is applied inside the same kernel."""
    return F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)


NORMS = "hip"   # the GPU norms: "hip" (the gfx950 kernels) or "torch" (the torch ops, as on the CPU)


def norm_modulate(x: Tensor, scale: Tensor, shift: Tensor, eps: float = 1e-6,
                  weight: Optional[Tensor] = None) -> Tensor:
    """The block's adaptive RMS norm ``rms_norm(x) * (1 + scale) + shift``: one gfx950 kernel on
    the GPU (``svdq::rms_norm_modulate``) unless ``NORMS`` is "torch", the torch ops elsewhere.
    ``weight``: ``1 + scale`` when the caller holds it already."""
    w = 1 + scale if weight is None else weight
    if x.is_cuda and NORMS == "hip":
        return hip_ops.rms_norm_modulate(x, w, shift, eps)
    return rms_norm(x, eps, weight=w) + shift


def residual_norm_modulate(x: Tensor, gate: Tensor, v: Tensor, scale: Tensor, shift: Tensor,
                           eps: float = 1e-6, weight: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """The gated residual ``x + gate * v`` (``torch.addcmul``, one bf16 rounding) and the adaptive
    RMS norm of the result: one gfx950 pass on the GPU (``svdq::residual_rms_norm_modulate``)
    unless ``NORMS`` is "torch".  Returns (new residual, normed activation)."""
    w = 1 + scale if weight is None else weight
    if x.is_cuda and NORMS == "hip":
        return hip_ops.residual_rms_norm_modulate(x, v, gate, w, shift, eps)
    x = torch.addcmul(x, gate, v)
    return x, norm_modulate(x, scale, shift, eps, weight=w)


def head_norm_rope(t: Tensor, cos: Tensor, sin: Tensor, eps: float = 1e-6) -> Tensor:
    """Per-head RMS norm of q or k [T, heads, head_dim] and the rotary embedding: one gfx950
    kernel on the GPU for head_dim 128 (``svdq::head_rms_rope``) unless ``NORMS`` is "torch",
    the torch ops elsewhere."""
    if t.is_cuda and NORMS == "hip":
        return hip_ops.head_rms_rope(t, cos, sin, eps)
    return apply_rope(rms_norm(t, eps), cos, sin)


GATES = "hip"   # the GPU sigmoid gate and SwiGLU product: "hip" (svdq::gate_op) or "torch"


def gate_mul_sigmoid(a: Tensor, g: Tensor) -> Tensor:
    """``a * sigmoid(g)`` in bf16 (torch's rounding): one gfx950 pass on the GPU unless ``GATES``
    is "torch"."""
    if a.is_cuda and GATES == "hip":
        return hip_ops.gate_op(g, a, hip_ops.EPILOGUES["mul_sigmoid"])
    return a * torch.sigmoid(g)


def gate_silu_mul(g: Tensor, u: Tensor) -> Tensor:
    """The SwiGLU product ``silu(g) * u`` in bf16 (torch's rounding): one gfx950 pass on the GPU
    unless ``GATES`` is "torch"."""
    if u.is_cuda and GATES == "hip":
        return hip_ops.gate_op(u, g, hip_ops.EPILOGUES["silu_mul"])
    return F.silu(g) * u


def rope_tables(tokens: int, head_dim: int, device, dtype, theta: float = 10000.0) -> tuple[Tensor, Tensor]:
    """cos / sin tables [tokens, head_dim] of the rotate-half rotary embedding."""
    inv = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim)
    ang = torch.arange(tokens, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def apply_rope(t: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """t [T, heads, d] rotated by position: t * cos + rotate_half(t) * sin, i.e. each pair
    (t1, t2) = (t[j], t[j + d/2]) -> (t1 c - t2 s, t2 c + t1 s), written half by half (no
    concatenated copy of rotate_half(t))."""
    d = t.shape[-1] // 2
    t1, t2 = t[..., :d], t[..., d:]
    c, s = cos[:, None, :d], sin[:, None, :d]       # the tables repeat their first half
    out = torch.empty_like(t)
    o1, o2 = out[..., :d], out[..., d:]
    torch.mul(t1, c, out=o1)
    o1.addcmul_(t2, s, value=-1)
    torch.mul(t2, c, out=o2)
    o2.addcmul_(t1, s)
    return out


LinearFn = Callable[[str, nn.Module, Tensor], Tensor]


def _module_linear(name: str, mod: nn.Module, x: Tensor) -> Tensor:
    return mod(x)


class _Attn(nn.Module):
    def __init__(self, layers: dict[str, nn.Module]):
        super().__init__()
        self.to_q, self.to_k, self.to_v = layers["attn.to_q"], layers["attn.to_k"], layers["attn.to_v"]
        self.to_gate = layers["attn.to_gate"]
        self.to_out = nn.ModuleList([layers["attn.to_out.0"]])


class _FF(nn.Module):
    def __init__(self, layers: dict[str, nn.Module]):
        super().__init__()
        self.gate, self.up, self.down = layers["ff.gate"], layers["ff.up"], layers["ff.down"]


class Krea2StandInBlock(nn.Module):
    """One block: the eight quantized linears (``attn.*``, ``ff.*``) plus modulation vectors."""

    def __init__(self, dims: Krea2Dims, layers: dict[str, nn.Module], modulation: Tensor):
        super().__init__()
        if set(layers) != set(LINEAR_NAMES):
            raise ValueError(f"block needs exactly the linears {LINEAR_NAMES}, got {sorted(layers)}")
        if tuple(modulation.shape) != (6, dims.hidden):
            raise ValueError(f"modulation must be [6, {dims.hidden}], got {tuple(modulation.shape)}")
        self.dims = dims
        self.attn = _Attn(layers)
        self.ff = _FF(layers)
        self.register_buffer("modulation", modulation.contiguous(), persistent=True)

    def linears(self) -> dict[str, nn.Module]:
        a, f = self.attn, self.ff
        return {"attn.to_q": a.to_q, "attn.to_k": a.to_k, "attn.to_v": a.to_v, "attn.to_gate": a.to_gate,
                "attn.to_out.0": a.to_out[0], "ff.gate": f.gate, "ff.up": f.up, "ff.down": f.down}

    def forward(self, x: Tensor, cos: Tensor, sin: Tensor, linear: LinearFn = _module_linear,
                modulation: Optional[Tensor] = None, fused: bool = False, siblings: bool | str = "grouped") -> Tensor:
        """x [T, hidden] -> [T, hidden].  ``linear(name, module, input)`` evaluates a quantized
        linear (default: the module itself); ``modulation`` overrides the block's buffer (a
        reference evaluation on another device passes its own copy).  ``fused=True`` runs the
        modules with the ops that follow to_gate, to_out.0, ff.up and ff.down fused into their
        kernels' stores (``SVDQuantLinear.forward_epilogue``: the same ops, the same bf16
        rounding); ``linear`` is then not used.  ``siblings`` groups the linears that read the
        same input (to_q, to_k, to_v, to_gate; ff.gate, ff.up): ``"grouped"`` (default) runs their
        GEMMs as one launch (``run_grouped``; with the default ``linear`` only), ``True`` or
        ``"concurrent"`` issues them concurrently on side streams (``run_concurrent``), ``False``
        one after another; all three give bit-identical outputs."""
        mod = self.modulation if modulation is None else modulation
        if fused:
            return self._forward_fused(x, cos, sin, self.linears(), tuple(m.to(x.dtype) for m in mod), siblings)
        x, (g_f, y_f) = self._forward_deferred(x, cos, sin, linear, mod, siblings, None)
        return torch.addcmul(x, g_f, y_f)

    def _norm_weights(self, mod: Tensor, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
        """``1 + scale`` of the two norms, computed once per modulation tensor (storage, version,
        dtype) instead of once per forward."""
        key = (mod.data_ptr(), mod._version, str(mod.device), dtype)
        hit = getattr(self, "_norm_w", None)
        if hit is None or hit[0] != key:
            hit = (key, (1 + mod[1].to(dtype), 1 + mod[4].to(dtype)))
            self._norm_w = hit
        return hit[1]

    def _forward_deferred(self, x: Tensor, cos: Tensor, sin: Tensor, linear: LinearFn, mod: Tensor,
                          siblings: bool | str, pending: Optional[tuple[Tensor, Tensor]]
                          ) -> tuple[Tensor, tuple[Tensor, Tensor]]:
        """The unfused block with its last gated residual left to the caller: returns ``(x, (g, y))``
        with the block output ``x + g * y``.  ``pending`` = the previous block's ``(g, y)``: its
        residual add is formed in the same pass as this block's first norm (one gfx950 kernel)."""
        d = self.dims
        shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = (m.to(x.dtype) for m in mod)
        w_a, w_f = self._norm_weights(mod, x.dtype)
        lin = self.linears()
        t = x.shape[0]

        def siblings_of(z: Tensor, *names: str) -> list[Tensor]:
            if siblings == "grouped" and linear is _module_linear:
                return run_grouped(z, [lin[n] for n in names])
            fns = [partial(linear, n, lin[n]) for n in names]
            if siblings is True or siblings == "concurrent":
                return run_concurrent(z, fns)
            return [f(z) for f in fns]

        if pending is None:
            h = norm_modulate(x, scale_a, shift_a, weight=w_a)
        else:
            x, h = residual_norm_modulate(x, pending[0], pending[1], scale_a, shift_a, weight=w_a)
        q, g, k, v = siblings_of(h, "attn.to_q", "attn.to_gate", "attn.to_k", "attn.to_v")
        q, k, v = (z.view(t, -1, d.head_dim) for z in (q, k, v))
        q = head_norm_rope(q, cos, sin)
        k = head_norm_rope(k, cos, sin)
        a = attention(q, k, v)                                   # [T, heads * head_dim]
        a = gate_mul_sigmoid(a, g)
        x, h = residual_norm_modulate(x, gate_a, linear("attn.to_out.0", lin["attn.to_out.0"], a), scale_f, shift_f,
                                      weight=w_f)
        u, g = siblings_of(h, "ff.up", "ff.gate")
        f = gate_silu_mul(g, u)
        return x, (gate_f, linear("ff.down", lin["ff.down"], f))

    def _forward_fused(self, x: Tensor, cos: Tensor, sin: Tensor, lin: dict, mods: tuple,
                       siblings: bool | str = "grouped") -> Tensor:
        """``forward`` with the gates, SwiGLU and residuals in the linears' epilogues (to_gate and
        ff.up then need the attention output and ff.gate's output: only to_q, to_k and to_v
        remain siblings)."""
        d = self.dims
        shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = mods
        t = x.shape[0]
        h = norm_modulate(x, scale_a, shift_a)
        fns = [lin["attn.to_q"], lin["attn.to_k"], lin["attn.to_v"]]
        if siblings == "grouped":
            q, k, v = run_grouped(h, fns)
        elif siblings is True or siblings == "concurrent":
            q, k, v = run_concurrent(h, fns)
        else:
            q, k, v = [f(h) for f in fns]
        q, k, v = (z.view(t, -1, d.head_dim) for z in (q, k, v))
        q = head_norm_rope(q, cos, sin)
        k = head_norm_rope(k, cos, sin)
        a = attention(q, k, v)
        a = lin["attn.to_gate"].forward_epilogue(h, "mul_sigmoid", aux=a)
        x = lin["attn.to_out.0"].forward_epilogue(a, "residual_gate", aux=x, vec=gate_a)
        h = norm_modulate(x, scale_f, shift_f)
        g = lin["ff.gate"](h)
        f = lin["ff.up"].forward_epilogue(h, "silu_mul", aux=g)
        return lin["ff.down"].forward_epilogue(f, "residual_gate", aux=x, vec=gate_f)


ATTENTION = "hip"   # the GPU attention: "hip" (svdq::attention) or "sdpa" (PyTorch's fused kernels)


def attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Softmax attention of q [T, H, d] over k, v [T, Hkv, d] (H a multiple of Hkv) -> [T, H*d].

    On the GPU with d = 128 the gfx950 kernel (``svdq::attention``) unless ``ATTENTION`` is
    "sdpa"; there only the fused SDPA kernels are allowed (flash / memory-efficient), the math
    path's batched products on transposed bf16 views are kept out.  Elsewhere (the CPU
    reference evaluation) SDPA picks its own path.
    """
    t, heads, dh = q.shape
    if q.is_cuda and dh == 128 and ATTENTION == "hip":
        return hip_ops.attention(q, k, v, 1.0 / math.sqrt(dh)).reshape(t, heads * dh)
    qh, kh, vh = (z.transpose(0, 1).unsqueeze(0) for z in (q, k, v))
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(qh, kh, vh, enable_gqa=True)
    else:
        o = F.scaled_dot_product_attention(qh, kh, vh, enable_gqa=True)
    return o.squeeze(0).transpose(0, 1).reshape(t, heads * dh)


class Krea2StandInTransformer(nn.Module):
    """``transformer_blocks`` of stand-in blocks; ``forward`` is one pass of the denoiser."""

    def __init__(self, dims: Krea2Dims, blocks: list[Krea2StandInBlock]):
        super().__init__()
        self.dims = dims
        self.transformer_blocks = nn.ModuleList(blocks)

    @classmethod
    def random(cls, dims: Krea2Dims = Krea2Dims(), *, rank: int = 32, group_size: int = 64,
               backend: str = "hip_gfx950", device: torch.device | str = "cuda", seed: int = 0
               ) -> "Krea2StandInTransformer":
        """Random-init model with every quantized linear resident on ``device``."""
        dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)
        blocks = []
        for _ in range(dims.layers):
            layers = {name: SVDQuantLinear(random_quantized_state(n, k, rank=rank, group_size=group_size,
                                                                  device=dev, generator=gen), backend=backend)
                      for name, (n, k) in dims.linear_shapes().items()}
            mod = torch.randn(6, dims.hidden, device=dev, generator=gen) * 0.1
            mod[2] = mod[2].abs() + 0.2   # attention gate
            mod[5] = mod[5].abs() + 0.2   # MLP gate
            blocks.append(Krea2StandInBlock(dims, layers, mod.to(torch.bfloat16)))
        return cls(dims, blocks)

    def forward(self, tokens: Tensor, linear: LinearFn = _module_linear, fused: bool = False,
                siblings: bool | str = "grouped") -> Tensor:
        """tokens [T, hidden] -> [T, hidden] through every block (``linear``, ``fused``,
        ``siblings`` as in the block)."""
        cos, sin = rope_tables(tokens.shape[0], self.dims.head_dim, tokens.device, tokens.dtype)
        x = tokens
        if fused:
            for blk in self.transformer_blocks:
                x = blk(x, cos, sin, linear, fused=True, siblings=siblings)
            return x
        # each block's last gated residual is formed with the next block's first norm
        pending = None
        for blk in self.transformer_blocks:
            x, pending = blk._forward_deferred(x, cos, sin, linear, blk.modulation, siblings, pending)
        return torch.addcmul(x, *pending)

    def denoise_step(self, text: Tensor, latent: Tensor, dt: float, fused: bool = False,
                     siblings: bool | str = "grouped") -> Tensor:
        """One Euler step of the flow: the denoiser over [text | latent], then
        ``latent + dt * velocity`` for the latent tokens."""
        out = self.forward(torch.cat([text, latent], dim=0), fused=fused, siblings=siblings)
        return latent + dt * out[text.shape[0]:]
