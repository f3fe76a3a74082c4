"""Offline conversion of a dense linear into the SVDQuant checkpoint layout (torch, any device).

This is the quantizer side of the format, not the forward path.  It follows the reference
recipe so that states built here are indistinguishable from reference checkpoints:

* ``quantize_symmetric_int4`` / ``dequantize_symmetric_int4`` / ``pack_int4`` /
  ``unpack_int4``: the group-wise symmetric INT4 format of reference ``quant/pack.py:6-70``
  (scale = amax.clamp_min(1e-8) / 7, codes = round-half-even(x / scale) clamped to [-8, 7],
  zero padding of K to a group multiple, low nibble = even index, offset +8);
* ``compute_smooth_scale`` (``quant/svd.py:26-30``), ``svd_lowrank`` (``quant/svd.py:33-86``);
* ``convert_linear``: migration, rank-r split, residual quantization and the storage dtypes
  of ``scripts/convert_simulated.py:184-208`` (packed uint8 codes, fp16 scales, bf16 smooth
  scale, bf16 low-rank factors, bf16 bias).

Running on a GPU keeps the randomized SVD and the quantization of large layers fast.
"""
from __future__ import annotations

import torch

from .state import SVDQuantLinearState


def quantize_symmetric_int4(x: torch.Tensor, group_size: int = 128, dim: int = -1):
    """Group-wise symmetric INT4; returns (int8 codes in [-8, 7], scales in x's dtype)."""
    k = x.shape[dim]
    if k % group_size:
        pad_shape = list(x.shape)
        pad_shape[dim] = group_size - k % group_size
        x = torch.cat([x, x.new_zeros(pad_shape)], dim=dim)
    moved = x.movedim(dim, -1).contiguous()
    lead = moved.shape[:-1]
    grouped = moved.reshape(*lead, moved.shape[-1] // group_size, group_size)
    scales = grouped.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 7.0
    codes = torch.round(grouped.float() / scales).clamp(-8, 7).to(torch.int8)
    codes = codes.reshape(moved.shape).movedim(-1, dim).contiguous()
    return codes, scales.squeeze(-1)


def dequantize_symmetric_int4(q: torch.Tensor, scales: torch.Tensor, group_size: int = 128,
                              dim: int = -1, dtype: torch.dtype | None = None) -> torch.Tensor:
    """``codes * scale`` per group, computed (and rounded) in ``dtype`` (default float32)."""
    dt = dtype or torch.float32
    moved = q.movedim(dim, -1).contiguous()
    lead = moved.shape[:-1]
    grouped = moved.reshape(*lead, moved.shape[-1] // group_size, group_size).to(dt)
    y = grouped * scales.unsqueeze(-1).to(dt)
    return y.reshape(moved.shape).movedim(-1, dim).contiguous()


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """Two signed INT4 codes per byte along the last dim: low nibble = even index, offset +8."""
    if q.dtype != torch.int8:
        raise TypeError("q must be torch.int8")
    if q.shape[-1] % 2:
        q = torch.cat([q, torch.zeros_like(q[..., :1])], dim=-1)
    u = (q.to(torch.int16) + 8).to(torch.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4)


def unpack_int4(packed: torch.Tensor, values_last_dim: int | None = None) -> torch.Tensor:
    """Inverse of ``pack_int4``: uint8 [..., B] -> int8 [..., 2B] (optionally truncated)."""
    if packed.dtype != torch.uint8:
        raise TypeError("packed must be torch.uint8")
    lo = (packed & 0x0F).to(torch.int8) - 8
    hi = ((packed >> 4) & 0x0F).to(torch.int8) - 8
    out = torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    return out if values_last_dim is None else out[..., :values_last_dim]


def compute_smooth_scale(x_absmax: torch.Tensor, weight: torch.Tensor,
                         min_value: float | None = 0.25, max_value: float | None = 4.0) -> torch.Tensor:
    """SmoothQuant migration scale ``sqrt(amax|X_:,j| / amax|W_:,j|)`` in the weight dtype.

    Clamped to ``[min_value, max_value]`` as in the reference; pass ``None`` for either bound
    to leave that side unclamped.
    """
    w_absmax = weight.abs().amax(dim=0).clamp_min(1e-8)
    s = torch.sqrt(x_absmax.float().clamp_min(1e-8) / w_absmax.float())
    if min_value is not None or max_value is not None:
        s = s.clamp(min_value, max_value)
    return s.to(weight.device, dtype=weight.dtype)


def svd_lowrank(weight: torch.Tensor, rank: int, *, oversample: int = 8, niter: int = 4,
                device: str | torch.device | None = None, exact: bool = False,
                seed: int | None = None):
    """Rank-r factors ``L1 = U_r diag(S_r)`` [out, r], ``L2 = V_r^T`` [r, in] of a 2-D weight."""
    if weight.ndim != 2:
        raise ValueError("svd_lowrank expects a 2D [out, in] weight")
    out_device, out_dtype = weight.device, weight.dtype
    w = weight.to(device=device if device is not None else out_device, dtype=torch.float32)
    min_dim = min(w.shape)
    rank = max(1, min(int(rank), min_dim))
    q = min(rank + max(0, int(oversample)), min_dim)
    if exact or min_dim <= max(q, 32):
        u, s, vh = torch.linalg.svd(w, full_matrices=False)
        u, s, vh = u[:, :rank], s[:rank], vh[:rank]
    else:
        if seed is not None:
            with torch.random.fork_rng(devices=[w.device] if w.is_cuda else []):
                torch.manual_seed(seed)
                u, s, v = torch.svd_lowrank(w, q=q, niter=max(0, int(niter)))
        else:
            u, s, v = torch.svd_lowrank(w, q=q, niter=max(0, int(niter)))
        u, s, vh = u[:, :rank], s[:rank], v[:, :rank].T
    l1 = (u * s.unsqueeze(0)).to(device=out_device, dtype=out_dtype).contiguous()
    l2 = vh.to(device=out_device, dtype=out_dtype).contiguous()
    return l1, l2


def convert_linear(weight: torch.Tensor, bias: torch.Tensor | None, x_absmax: torch.Tensor | None, *,
                   rank: int = 32, group_size: int = 64,
                   smooth_clamp: tuple[float | None, float | None] = (0.25, 4.0),
                   oversample: int = 8, niter: int = 4, exact_svd: bool = False,
                   seed: int | None = None) -> SVDQuantLinearState:
    """Quantize one dense linear [N, K] into the packed checkpoint layout.

    ``x_absmax=None`` gives identity smoothing (the reference's uncalibrated conversion).  The
    smoothing scale is rounded to bf16 first and the migration uses that stored value; the
    migrated weight ``W * s`` is rounded to the weight's own dtype, as the reference converter
    does for its bf16 weights (``convert_simulated.py:188-194``; a no-op for fp32 weights), and
    the residual subtracts the bf16-rounded factors that the runtime will use.
    """
    if weight.ndim != 2:
        raise ValueError("linear weight must be [out_features, in_features]")
    n, k = weight.shape
    w = weight.float()
    if x_absmax is None:
        smooth = torch.ones(k, device=w.device, dtype=torch.bfloat16)
    else:
        smooth = compute_smooth_scale(x_absmax.to(w.device), w, *smooth_clamp).to(torch.bfloat16)
    migrated = (w * smooth.float().unsqueeze(0)).to(weight.dtype).float()
    l1, l2 = svd_lowrank(migrated, rank, oversample=oversample, niter=niter, exact=exact_svd, seed=seed)
    l1, l2 = l1.to(torch.bfloat16), l2.to(torch.bfloat16)
    residual = migrated - l1.float() @ l2.float()
    q, scales = quantize_symmetric_int4(residual, group_size=group_size, dim=1)
    packed = pack_int4(q)
    return SVDQuantLinearState(
        smooth_scale=smooth.contiguous(),
        qweight=packed.contiguous(),
        weight_scales=scales.to(torch.float16).contiguous(),
        l1=l1.contiguous(),
        l2=l2.contiguous(),
        bias=None if bias is None else bias.detach().to(torch.bfloat16).contiguous(),
        group_size=int(group_size),
        original_shape=(int(n), int(k)),
        qweight_packed=True,
        padded_in_features=int(packed.shape[1]) * 2,
    )


def quantize_linear_from_samples(weight: torch.Tensor, bias: torch.Tensor | None, x_samples: torch.Tensor,
                                 rank: int = 32, group_size: int = 128, smooth_min: float = 0.25,
                                 smooth_max: float = 4.0) -> SVDQuantLinearState:
    """Reference-named entry (``quant/svd.py:89-116``) producing the packed checkpoint layout."""
    x_absmax = x_samples.float().abs().amax(dim=0)
    return convert_linear(weight, bias, x_absmax, rank=rank, group_size=group_size,
                          smooth_clamp=(smooth_min, smooth_max))
