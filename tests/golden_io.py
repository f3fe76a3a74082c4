"""Loading of the committed golden fixtures into oracle states (shared by CPU and GPU tests)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import numerics as nm
from oracle import sim


def load_layer_fixture(path: Path):
    fx = dict(np.load(path))
    x = nm.from_bf16_bits(fx["x"])
    st = sim.LayerState(
        smooth=nm.from_bf16_bits(fx["smooth"]), qweight=fx["qweight"],
        weight_scales=fx["weight_scales"].astype(np.float32), l1=nm.from_bf16_bits(fx["l1"]),
        l2=nm.from_bf16_bits(fx["l2"]), bias=nm.from_bf16_bits(fx["bias"]),
        group_size=int(fx["group_size"]), shape=(fx["qweight"].shape[0], fx["x"].shape[1]),
        adapters=[sim.Adapter(down=nm.from_bf16_bits(fx["lora_down"]), up=nm.from_bf16_bits(fx["lora_up"]),
                              scale=float(fx["lora_scale"]), network_alpha=float(fx["lora_alpha"]))])
    return fx, x, st
