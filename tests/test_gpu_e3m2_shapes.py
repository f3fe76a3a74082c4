"""GPU parity of the production W4A4 path (e3m2 operands on the FP6 MFMA, the default) at the
benchmark shapes: config 0, the config 1 shapes at M=4096 (ff.up, ff.down with K=16384, to_k with
N=1536) and config 4 (M=16384, ff.up and ff.down with a rank-64 LoRA on the rank-32 branch); and an
activation operand of more than 2^31 elements on both tilings (M=131200 / 131328, K=16384).

Bars: the e3m2 activation operand (decoded through the format definition, independently of the
encoder) and the sx pairs bit-exact against the oracle quantizer; layer outputs in float32 mode
within relative L2 1e-4 of the float64 evaluation of the quantized math, bf16 outputs within 1e-3
of bf16(oracle) (1e-3 is the tolerance allowed for both); and, over whole outputs, the exact
power-of-two homogeneity y(2x) - b = 2 (y(x) - b).  Large layers are built on the GPU by the
package converter and checked on a row sample (every row of x is quantized and multiplied
independently).
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim, synth
from tests.gpu_util import (bf16_tensor, device_adapters, e3m2_codes_of, from_device_state, rel_l2,
                            sx_pairs_ok, to_device_state)

pytestmark = pytest.mark.gpu
TOL, TOL_F32 = 1e-3, 1e-4


def _gpu_layer(dev, m, k, n, seed, bias=True):
    """x bf16 [m, k] ~ N(0,1) with 1% outlier channels x20, and a layer converted on the GPU from
    W ~ N(0, 0.02) (rank 32, group 64, unclamped smoothing), as bench.py builds them."""
    from krea2_svdquant_amd.quant.convert import convert_linear
    gen = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(m, k, device=dev, generator=gen)
    x[:, torch.randperm(k, device=dev, generator=gen)[: round(0.01 * k)]] *= 20.0
    x = x.to(torch.bfloat16)
    w = torch.randn(n, k, device=dev, generator=gen) * 0.02
    b = torch.randn(n, device=dev, generator=gen) * 0.1 if bias else None
    ds = convert_linear(w, b, x.float().abs().amax(0), rank=32, group_size=64, smooth_clamp=(None, None),
                        seed=seed + 2)
    del w
    return x, ds


def _rows(m, count, seed):
    rows = np.sort(np.random.default_rng(seed).choice(m, count, replace=False))
    rows[0], rows[-1] = 0, m - 1          # the first and last row of the operand
    return np.unique(rows)


def _check_codes(dev, x, prep, st, rows=None):
    """The e3m2 operand and sx pairs of act_quant (the production flags) against the oracle."""
    from krea2_svdquant_amd.kernels.hip import ops
    qa, sxp, _, _, _ = ops.act_quant(x, prep.srs, prep.l2, prep.lora_down, prep.lora_mult, 64, prep.rtp,
                                     ops.OPERAND_E3M2, False, False, False, True)
    xs = x if rows is None else x[torch.from_numpy(rows).to(dev)]
    _, _, sx_ref, codes = sim.quantize_activations(xs.float().cpu().numpy(), st)
    got = e3m2_codes_of(qa.cpu().numpy(), x.shape[0], x.shape[1], rows)
    assert np.array_equal(got, codes), f"{int((got != codes).sum())} e3m2 codes differ"
    assert sx_pairs_ok(sxp, sx_ref, rows)


def _check_rows(dev, x, prep, st, rows, tag):
    from krea2_svdquant_amd.kernels.hip import backend
    ridx = torch.from_numpy(rows).to(dev)
    ref = sim.w4a4_eval(x[ridx].float().cpu().numpy(), st)["y"]
    y32 = backend.forward_prepared(x, prep, mode="w4a4", out_f32=True)
    e32 = rel_l2(y32[ridx].cpu().numpy(), ref)
    y16 = backend.forward_prepared(x, prep, mode="w4a4")
    e16 = rel_l2(y16[ridx].float().cpu().numpy(), nm.bf16(ref.astype(np.float32)))
    print(f"  {tag}: {len(rows)} rows, rel_l2 f32-out={e32:.3e} bf16-out vs bf16(ref)={e16:.3e}")
    assert e32 < TOL_F32 and e16 < TOL
    return y32


def _check_homogeneity(dev, x, prep, y, bias):
    from krea2_svdquant_amd.kernels.hip import backend
    y2 = backend.forward_prepared(x * 2, prep, mode="w4a4", out_f32=True)
    b = bias.float() if bias is not None else torch.zeros((), device=dev)
    hom = ((y2 - b) - 2 * (y - b)).norm() / (y - b).norm()
    assert hom.item() < 1e-6, hom.item()


def test_config0_e3m2(dev):
    """Config 0 (M=256, K=N=6144, rank 32, g64, outliers), every row and code."""
    from krea2_svdquant_amd.kernels.hip import backend
    x = synth.make_activation(256, 6144, seed=0)
    st = synth.make_layer(6144, 6144, x, rank=32, group_size=64, seed=1)
    prep = backend.prepare_layer(to_device_state(st, dev), (), dev)
    xd = bf16_tensor(x, dev)
    _check_codes(dev, xd, prep, st)
    _check_rows(dev, xd, prep, st, np.arange(256), "config0 e3m2")


@pytest.mark.parametrize("name,n,k", [("ff.up", 16384, 6144), ("ff.down", 6144, 16384), ("to_k", 1536, 6144)])
def test_config1_shapes_e3m2(dev, name, n, k):
    """Config 1 shapes at M=4096: every code and sx pair; 48 sampled output rows; homogeneity
    over the whole output."""
    from krea2_svdquant_amd.kernels.hip import backend
    m = 4096
    x, ds = _gpu_layer(dev, m, k, n, seed=k + n)
    prep = backend.prepare_layer(ds, (), dev)
    st = from_device_state(ds)
    _check_codes(dev, x, prep, st)
    y = _check_rows(dev, x, prep, st, _rows(m, 48, 7), f"config1 {name} e3m2")
    _check_homogeneity(dev, x, prep, y, ds.bias)


@pytest.mark.parametrize("name,n,k", [("ff.up", 16384, 6144), ("ff.down", 6144, 16384)])
def test_config4_lora_e3m2(dev, name, n, k):
    """Config 4: M=16384 (batch 4 at 1024px), rank-32 SVD branch plus a rank-64 LoRA
    (A, B ~ N(0, 0.01), scale 0.8) fused; codes, sx pairs and outputs on a row sample."""
    from krea2_svdquant_amd.kernels.hip import backend
    m = 16384
    x, ds = _gpu_layer(dev, m, k, n, seed=3 * k + n, bias=False)
    st = from_device_state(ds)
    st.adapters.append(synth.make_adapter(n, k, rank=64, std=0.01, scale=0.8, seed=4))
    prep = backend.prepare_layer(ds, device_adapters(st, dev), dev)
    assert prep.rtp == 96
    rows = _rows(m, 40, 9)
    _check_codes(dev, x, prep, st, rows)
    y = _check_rows(dev, x, prep, st, rows, f"config4 {name} e3m2 + LoRA r64")
    _check_homogeneity(dev, x, prep, y, None)    # the LoRA branch (on raw x) is linear in x too


@pytest.mark.parametrize("m,n", [(131200, 256), (131328, 512)])
def test_large_rows_e3m2(dev, m, n):
    """An activation operand of more than 2^31 elements (K=16384): the e3m2 codes, sx pairs and
    outputs of sampled rows, the last ones included, against the oracle (M=131200 takes the
    256 x 128 tiles, M=131328 with N=512 the 256 x 256 tiles)."""
    from krea2_svdquant_amd.kernels.hip import backend, lib, ops
    k = 16384
    assert m * k > 2 ** 31
    cols = lib.w4a4_tile_cols(m, n, k, 64, ops.OPERAND_E3M2)
    print(f"e3m2 with M*K > 2^31: M={m} K={k} N={n}, tile columns {cols}", flush=True)
    assert cols == (256 if m % 256 == 0 else 128)
    x, ds = _gpu_layer(dev, m, k, n, seed=m + n)
    prep = backend.prepare_layer(ds, (), dev)
    st = from_device_state(ds)
    rows = np.unique(np.concatenate([_rows(m, 16, 5), np.arange(m - 8, m)]))
    _check_codes(dev, x, prep, st, rows)
    _check_rows(dev, x, prep, st, rows, f"M={m} e3m2")


@pytest.mark.parametrize("m,k,g", [(1, 64, 64), (5, 448, 64), (64, 1024, 64), (100, 768, 128), (257, 1536, 64),
                                   (600, 6144, 64), (3, 16384, 64)])
def test_act_quant_random_shapes_e3m2_bit_exact(dev, m, k, g):
    """The production activation flags (e3m2 planar operand + sx pairs) on ragged shapes."""
    from krea2_svdquant_amd.kernels.hip import backend
    x = synth.make_activation(m, k, seed=m + k)
    st = synth.make_layer(64, k, x, rank=32, group_size=g, seed=3)
    prep = backend.prepare_layer(to_device_state(st, dev), (), dev)
    from krea2_svdquant_amd.kernels.hip import ops
    xd = bf16_tensor(x, dev)
    qa, sxp, _, _, _ = ops.act_quant(xd, prep.srs, prep.l2, None, None, g, prep.rtp, ops.OPERAND_E3M2, False,
                                     False, False, True)
    _, _, sx_ref, codes = sim.quantize_activations(x, st)
    assert np.array_equal(e3m2_codes_of(qa.cpu().numpy(), m, k), codes)
    assert sx_pairs_ok(sxp, sx_ref)
