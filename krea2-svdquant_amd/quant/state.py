"""``SVDQuantLinearState``: the per-layer tensors of the checkpoint layout.

Same fields and meaning as reference ``src/krea2_svdquant/quant/svd.py:12-23``; the kernels
of this package read the packed layout (``qweight_packed=True``) that
``runtime/load.py:106-125`` builds from ``transformer_svdquant.safetensors``:

* ``smooth_scale``  bf16 [K]
* ``qweight``       uint8 [N, Kp/2], byte j = (q[2j]+8) | (q[2j+1]+8) << 4
* ``weight_scales`` fp16 [N, Kp/G]
* ``l1``            bf16 [N, r];  ``l2`` bf16 [r, K];  ``bias`` bf16 [N] or None
* ``group_size``, ``original_shape=(N, K)``, ``padded_in_features=Kp``
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class SVDQuantLinearState:
    smooth_scale: torch.Tensor
    qweight: torch.Tensor
    weight_scales: torch.Tensor
    l1: torch.Tensor
    l2: torch.Tensor
    bias: torch.Tensor | None
    group_size: int
    original_shape: tuple[int, int]
    qweight_packed: bool = False
    padded_in_features: int | None = None
