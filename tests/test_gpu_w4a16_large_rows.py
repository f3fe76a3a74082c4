"""GPU parity of the W4A16 path for an activation operand above 4 GiB (M = 131200, K = 16384).

The 192-row tiles' specialized-wave kernel (``w4a16_ws_kernel``) addresses x_hat rows by a 32-bit
byte offset from the operand's base (row * K * 2), which cannot reach rows past 2^31 / K; for such
shapes the launcher takes the register-staged kernel, which addresses rows in 64 bits.  This shape
(N = 256: 192-row tiles chosen) would otherwise run the specialized kernel.  Rows are sampled across
the whole operand, the last ones beyond the 4 GiB offset, and checked against the oracle's
``w4a16_eval`` (the reference pytorch_sim forward, ``quant/svd.py:119-163``; dequantization
``quant/pack.py:26-44``) within relative L2 1e-4 (float32 out), plus x_hat bit-exact on those rows.
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim
from oracle.pack import smooth_activations
from tests.gpu_util import bf16_bits_of, from_device_state, rel_l2

pytestmark = pytest.mark.gpu


def test_w4a16_rows_beyond_4gib(dev):
    from krea2_svdquant_amd.kernels.hip import backend, ops
    from krea2_svdquant_amd.quant.convert import convert_linear
    m, k, n = 131200, 16384, 256
    assert (m - 1) * k * 2 >= 2 ** 32
    print(f"W4A16 with x_hat above 4 GiB: M={m} K={k} N={n}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(17)
    x = torch.randn(m, k, device=dev, generator=gen, dtype=torch.bfloat16)
    w = torch.randn(n, k, device=dev, generator=gen) * 0.02
    b = torch.randn(n, device=dev, generator=gen) * 0.1
    ds = convert_linear(w, b, x[:4096].float().abs().amax(0), rank=32, group_size=64, smooth_clamp=(None, None),
                        seed=19)
    del w
    prep = backend.prepare_layer(ds, (), dev)
    st = from_device_state(ds)

    rows = np.unique(np.concatenate([[0, 1, m // 2], np.arange(m - 8, m),
                                     np.random.default_rng(3).choice(m, 16, replace=False)]))
    ridx = torch.from_numpy(rows).to(dev)
    xs = x[ridx].float().cpu().numpy()

    _, _, _, xhat, _ = ops.act_quant(x, prep.srs, prep.l2, None, None, 64, prep.rtp, ops.OPERAND_NONE, False,
                                     True, False)
    assert np.array_equal(bf16_bits_of(xhat[ridx]), nm.bf16_bits(smooth_activations(xs, st.smooth)))
    del xhat

    y = backend.forward_prepared(x, prep, mode="w4a16", out_f32=True)
    torch.cuda.synchronize()
    ref = sim.w4a16_eval(xs, st)["y"]
    e = rel_l2(y[ridx].cpu().numpy(), ref)
    e_last = rel_l2(y[ridx[-8:]].cpu().numpy(), ref[-8:]) if rows[-1] == m - 1 else e
    print(f"  {len(rows)} rows: rel_l2 f32-out={e:.3e}, last 8 rows {e_last:.3e}", flush=True)
    assert torch.isfinite(y).all()
    assert e < 1e-4 and e_last < 1e-4
