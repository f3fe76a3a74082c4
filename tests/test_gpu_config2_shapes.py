"""GPU parity of the W4A16 path at benchmark config 2's own shapes: M=2304 (768x768 latent), the
four distinct (N, K) shapes of a Krea-2 block's eight linears (to_q / to_gate / to_out.0
6144->6144, to_k / to_v 6144->1536, ff.gate / ff.up 6144->16384, ff.down 16384->6144), rank 32,
group 64, outlier activations, layers converted on the GPU as bench.py builds them.

This reaches the one-wave-per-SIMD wide kernel's long-K main loop at K=6144 and K=16384 (ff.up,
ff.down, to_q) and the 128x128 kernel (to_k at N=1536).  The math is the reference pytorch_sim
forward (``quant/svd.py:119-163``; dequantization ``quant/pack.py:26-44``).

Bars: x_hat bit-exact against the oracle's smoothing on every row; layer outputs on a row sample
within relative L2 1e-4 of the float64 evaluation of the sim's bf16 operands in float32 mode and
within 1e-3 of bf16(oracle) in bf16 mode; over the whole output, the exact power-of-two
homogeneity y(2x) - b = 2 (y(x) - b) (x_hat, both GEMMs and the low-rank operand scale exactly
by 2).
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim
from oracle.pack import smooth_activations
from tests.gpu_util import bf16_bits_of, from_device_state, rel_l2

pytestmark = pytest.mark.gpu
TOL, TOL_F32 = 1e-3, 1e-4
M = 2304


def _gpu_layer(dev, m, k, n, seed, bias=True):
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
    rows[0], rows[-1] = 0, m - 1
    return np.unique(rows)


@pytest.mark.parametrize("name,n,k", [("to_q", 6144, 6144), ("to_k", 1536, 6144), ("ff.up", 16384, 6144),
                                      ("ff.down", 6144, 16384)])
def test_config2_w4a16_shapes(dev, name, n, k):
    from krea2_svdquant_amd.kernels.hip import backend, ops
    print(f"config2 W4A16 {name}: M={M} K={k} N={n}", flush=True)
    x, ds = _gpu_layer(dev, M, k, n, seed=5 * k + n)
    prep = backend.prepare_layer(ds, (), dev)
    st = from_device_state(ds)

    # x_hat of the production W4A16 flags, every row, bit for bit
    _, _, _, xhat, _ = ops.act_quant(x, prep.srs, prep.l2, None, None, 64, prep.rtp, ops.OPERAND_NONE, False,
                                     True, False)
    xh_ref = smooth_activations(x.float().cpu().numpy(), st.smooth)
    assert np.array_equal(bf16_bits_of(xhat), nm.bf16_bits(xh_ref)), "x_hat differs from the oracle"

    rows = _rows(M, 48, 11)
    ridx = torch.from_numpy(rows).to(dev)
    ref = sim.w4a16_eval(x[ridx].float().cpu().numpy(), st)["y"]
    y32 = backend.forward_prepared(x, prep, mode="w4a16", out_f32=True)
    y16 = backend.forward_prepared(x, prep, mode="w4a16")
    e32 = rel_l2(y32[ridx].cpu().numpy(), ref)
    e16 = rel_l2(y16[ridx].float().cpu().numpy(), nm.bf16(ref.astype(np.float32)))
    print(f"  {len(rows)} rows: rel_l2 f32-out={e32:.3e} bf16-out vs bf16(ref)={e16:.3e}", flush=True)
    assert e32 < TOL_F32 and e16 < TOL

    # the bf16 output is the bf16 rounding of the float32 one (same kernel, one rounding at the store)
    assert torch.equal(y16, y32.to(torch.bfloat16))

    y2 = backend.forward_prepared(x * 2, prep, mode="w4a16", out_f32=True)
    b = ds.bias.float() if ds.bias is not None else torch.zeros((), device=dev)
    hom = ((y2 - b) - 2 * (y32 - b)).norm() / (y32 - b).norm()
    assert hom.item() < 1e-6, hom.item()
