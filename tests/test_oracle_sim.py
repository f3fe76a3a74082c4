"""Pins the oracle's layer evaluators (oracle/sim.py, oracle/synth.py).

Checks used:
* the reference's LoRA known answer (tests/test_lora_loading.py:39-63, via golden data):
  multiplier 0.5 * 4 / 2 = 1.0 and up(down(x)) on the raw x;
* brute force: explicit loops over m, n, groups and k with exact integer group sums;
* the sim restatement against the float64 W4A16 evaluator (same math, bf16 roundings only);
* W4A4 against W4A16 (activation quantization error of a 4-bit grid, bounded);
* the reference's sim shape test (tests/test_svd_linear_cpu.py:6-13);
* regression against the committed fixtures.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import pack as op
from oracle import sim, synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_lora_known_answer():
    ka = json.loads((GOLDEN / "reference_known_answers.json").read_text())["lora"]
    down, up, x = (np.array(ka[k]) for k in ("down", "up", "x"))
    ad = sim.Adapter(down=down.astype(np.float32), up=up.astype(np.float32), scale=ka["scale"],
                     network_alpha=ka["alpha"])
    assert ad.multiplier == ka["multiplier"] == 1.0
    # a layer whose quantized part is exactly zero: codes 0 (bytes 0x88), zero low-rank factors
    st = sim.LayerState(smooth=np.ones(4, np.float32), qweight=np.full((3, 2), 0x88, np.uint8),
                        weight_scales=np.ones((3, 1), np.float32), l1=np.zeros((3, 1), np.float32),
                        l2=np.zeros((1, 4), np.float32), bias=None, group_size=4, shape=(3, 4),
                        adapters=[sim.Adapter(down=nm.bf16(down.astype(np.float32)), up=nm.bf16(up.astype(np.float32)),
                                              scale=ka["scale"], network_alpha=ka["alpha"])])
    xb = nm.bf16(x.astype(np.float32))
    expect = (xb.astype(np.float64) @ nm.bf16(down.astype(np.float32)).T.astype(np.float64)) @ \
        nm.bf16(up.astype(np.float32)).T.astype(np.float64)
    for ev in (sim.w4a4_eval, sim.w4a16_eval):
        np.testing.assert_allclose(ev(xb, st)["y"], expect, rtol=1e-12, atol=1e-12)
    # the un-rounded reference numbers agree to bf16 precision of the inputs
    np.testing.assert_allclose(expect, np.array(ka["expected"]), rtol=2e-2, atol=2e-2)


def _bruteforce_w4a4(x, st):
    xh = op.smooth_activations(x, st.smooth)
    m, k = x.shape
    n = st.shape[0]
    g = st.group_size
    qw = st.weight_codes()
    y = np.zeros((m, n))
    for i in range(m):
        row = xh[i]
        for gi in range(k // g):
            seg = row[gi * g:(gi + 1) * g]
            amax = max(abs(float(v)) for v in seg)
            sc = float(nm.bf16(np.float32(max(amax, nm.BF16_1E_8)) / np.float32(7.0)))
            codes = [int(np.clip(np.rint(np.float32(v) / np.float32(sc)), -8, 7)) for v in seg]
            for j in range(n):
                acc = sum(codes[t] * int(qw[j, gi * g + t]) for t in range(g))
                y[i, j] += sc * float(st.weight_scales[j, gi]) * acc
    mid = [[sum(float(xh[i, t]) * float(st.l2[c, t]) for t in range(k)) for c in range(st.l2.shape[0])] for i in range(m)]
    for i in range(m):
        for j in range(n):
            y[i, j] += sum(mid[i][c] * float(st.l1[j, c]) for c in range(st.l1.shape[1]))
            if st.bias is not None:
                y[i, j] += float(st.bias[j])
    return y


def test_w4a4_eval_matches_bruteforce():
    x = synth.make_activation(3, 128, seed=5)
    st = synth.make_layer(5, 128, x, rank=4, group_size=64, seed=6, bias=True)
    np.testing.assert_allclose(sim.w4a4_eval(x, st)["y"], _bruteforce_w4a4(x, st), rtol=1e-10, atol=1e-10)


def test_sim_restatement_vs_float64_w4a16():
    x = synth.make_activation(64, 512, seed=7)
    st = synth.make_layer(384, 512, x, rank=32, group_size=64, seed=8, bias=True)
    st.adapters.append(synth.make_adapter(384, 512, rank=16, seed=9))
    y_sim = sim.sim_forward_torch(torch.from_numpy(x).to(torch.bfloat16), st).float().numpy()
    ref = sim.w4a16_eval(x, st)["y"]
    # bf16 outputs of three GEMMs and two adds: a few bf16 ulps
    assert sim.rel_l2(y_sim, ref) < 1e-2
    # W4A4 differs by the activation quantization error only (4-bit grid, outliers smoothed)
    assert 1e-3 < sim.rel_l2(sim.w4a4_eval(x, st)["y"], ref) < 0.2


def test_reference_sim_shape_case():
    x = nm.bf16(torch.randn(8, 32, generator=torch.Generator().manual_seed(0)).numpy())
    st = synth.make_layer(16, 32, x, rank=4, group_size=16, seed=0)
    y = sim.sim_forward_torch(torch.from_numpy(x).to(torch.bfloat16), st)
    assert tuple(y.shape) == (8, 16) and torch.isfinite(y.float()).all()


@pytest.mark.parametrize("name", ["w4a4_small_g64.npz", "w4a4_small_g128.npz"])
def test_fixture_regression(name):
    from tests.golden_io import load_layer_fixture
    fx, x, st = load_layer_fixture(GOLDEN / name)
    r4 = sim.w4a4_eval(x, st)
    assert np.array_equal(nm.bf16_bits(r4["x_hat"]), fx["xhat"])
    assert np.array_equal(r4["qx_packed"], fx["qx_packed"])
    assert np.array_equal(nm.bf16_bits(r4["sx"]), fx["sx"])
    np.testing.assert_allclose(r4["y"], fx["y_w4a4"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sim.w4a16_eval(x, st)["y"], fx["y_w4a16"], rtol=1e-12, atol=1e-12)


def test_edge_activation_fixture_regression():
    fx = np.load(GOLDEN / "edge_activations.npz")
    x = nm.from_bf16_bits(fx["x"])
    s = nm.from_bf16_bits(fx["smooth"])
    xh = op.smooth_activations(x, s)
    packed, sx, q = op.quantize_activations_a4(xh, 64)
    assert np.array_equal(nm.bf16_bits(xh), fx["xhat"])
    assert np.array_equal(packed, fx["qx_packed"]) and np.array_equal(nm.bf16_bits(sx), fx["sx"])
    assert q[1, :8].tolist() == [7, 2, 4, -2, 0, 2, -7, 0]


@pytest.mark.parametrize("m,k,g", [(37, 448, 64), (16, 1024, 128), (64, 6144, 64)])
def test_torch_a4_quantizer_matches_numpy_restatement(m, k, g):
    """The torch restatement (the multithreaded CPU baseline) gives the numpy oracle's bits."""
    import torch
    from oracle import numerics as nm
    x = synth.make_activation(m, k, seed=m)
    st = synth.make_layer(32, k, x, rank=8, group_size=g, seed=2)
    xt = torch.from_numpy(nm.bf16_bits(x).view(np.int16)).view(torch.bfloat16)
    packed, scales = sim.quantize_activations_torch(xt, st)
    _, packed_ref, sx_ref, _ = sim.quantize_activations(x, st)
    assert np.array_equal(packed.numpy(), packed_ref)
    assert np.array_equal(scales.view(torch.int16).numpy().view(np.uint16), nm.bf16_bits(sx_ref))
