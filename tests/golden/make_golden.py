"""Writes the committed golden fixtures of tests/golden/ (run from the repo root).

* reference_known_answers.json -- data of the reference's own known-answer tests:
  - tests/test_pack.py:6-10: codes arange(-8, 8) x 3 rows round-trip through pack/unpack;
    the packed bytes listed follow from the layout byte j = (q[2j]+8) | (q[2j+1]+8) << 4;
  - tests/test_lora_loading.py:39-63: down = arange(8).reshape(2, 4) / 10,
    up = arange(6).reshape(3, 2) / 10, alpha 4, scale 0.5 -> multiplier 0.5 * 4 / 2 = 1.0,
    output = up(down(x)) * 1.0 on the raw x (a fixed x replaces the test's randn).
* w4a4_small_g{64,128}.npz -- small seeded layers (bias, one LoRA adapter, K not a multiple of
  the GEMM tile) with the oracle's x_hat, packed codes, scales, mid and float64 outputs of the
  W4A4 and W4A16 math; and edge_activations.npz -- activation rows exercising zero groups,
  exact .5 ties, tiny and huge magnitudes.

The fixtures are produced by the oracle (oracle/), whose functions are pinned by
tests/test_oracle_pack.py and tests/test_oracle_sim.py; the GPU tests compare against them.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import numerics as nm  # noqa: E402
from oracle import pack as op  # noqa: E402
from oracle import sim, synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def known_answers() -> dict:
    codes = np.tile(np.arange(-8, 8, dtype=np.int8), (3, 1))
    down = np.arange(8, dtype=np.float64).reshape(2, 4) / 10
    up = np.arange(6, dtype=np.float64).reshape(3, 2) / 10
    x = np.array([[0.5, -1.0, 2.0, 0.25], [-0.75, 1.5, 0.0, -2.0]])
    mult = 0.5 * 4.0 / 2
    return {
        "pack_roundtrip": {"codes": codes.tolist(), "packed": op.pack_int4(codes).tolist(),
                           "source": "reference tests/test_pack.py:6-10"},
        "lora": {"down": down.tolist(), "up": up.tolist(), "alpha": 4.0, "scale": 0.5, "multiplier": mult,
                 "x": x.tolist(), "expected": ((x @ down.T) @ up.T * mult).tolist(),
                 "source": "reference tests/test_lora_loading.py:39-63"},
    }


def layer_fixture(group: int, seed: int) -> dict:
    m, k, n, r = 37, 320 if group == 64 else 384, 96, 8
    x = synth.make_activation(m, k, seed=seed)
    st = synth.make_layer(n, k, x, rank=r, group_size=group, seed=seed + 1, bias=True)
    st.adapters.append(synth.make_adapter(n, k, rank=4, std=0.05, scale=0.8, network_alpha=2.0, seed=seed + 2))
    r4 = sim.w4a4_eval(x, st)
    r16 = sim.w4a16_eval(x, st)
    ad = st.adapters[0]
    return dict(
        x=nm.bf16_bits(x), smooth=nm.bf16_bits(st.smooth), qweight=st.qweight,
        weight_scales=st.weight_scales.astype(np.float16), l1=nm.bf16_bits(st.l1), l2=nm.bf16_bits(st.l2),
        bias=nm.bf16_bits(st.bias), lora_down=nm.bf16_bits(ad.down), lora_up=nm.bf16_bits(ad.up),
        lora_scale=np.float64(ad.scale), lora_alpha=np.float64(ad.network_alpha), group_size=np.int64(group),
        xhat=nm.bf16_bits(r4["x_hat"]), qx_packed=r4["qx_packed"], sx=nm.bf16_bits(r4["sx"]),
        mid=r4["mid"], y_w4a4=r4["y"], y_w4a16=r16["y"],
    )


def edge_activations() -> dict:
    k = 256
    rows = []
    rows.append(np.zeros(k))                                   # all-zero groups
    t = np.zeros(k)
    t[:8] = [7.0, 2.5, 3.5, -2.5, -0.5, 1.5, -7.0, 0.5]       # exact ties with s = 1
    t[64:72] = [14.0, 5.0, 7.0, -5.0, -1.0, 3.0, -14.0, 1.0]  # ties at scale 2
    rows.append(t)
    rows.append(np.full(k, 1e-35))                             # tiny groups (slow path)
    rows.append(np.full(k, -3e35))                             # huge groups (slow path)
    mixed = np.random.default_rng(9).standard_normal(k)
    mixed[:64] *= 1e-38                                        # subnormal-range values
    mixed[64:128] *= 1e30
    rows.append(mixed)
    rows.append(np.where(np.arange(k) % 2 == 0, -0.0, 3.0))    # signed zeros
    x = nm.bf16(np.array(rows, dtype=np.float32))
    s = np.ones(k, np.float32)
    s[128:] = nm.bf16(np.float32(1.5))
    xh = op.smooth_activations(x, s)
    packed, sx, _ = op.quantize_activations_a4(xh, 64)
    return dict(x=nm.bf16_bits(x), smooth=nm.bf16_bits(s), xhat=nm.bf16_bits(xh), qx_packed=packed,
                sx=nm.bf16_bits(sx))


def main() -> None:
    (OUT / "reference_known_answers.json").write_text(json.dumps(known_answers(), indent=1))
    np.savez_compressed(OUT / "w4a4_small_g64.npz", **layer_fixture(64, 10))
    np.savez_compressed(OUT / "w4a4_small_g128.npz", **layer_fixture(128, 20))
    np.savez_compressed(OUT / "edge_activations.npz", **edge_activations())
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
