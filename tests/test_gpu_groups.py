"""GPU parity for group sizes other than 64 / 128 (the generic kernels): any multiple of 16 that
divides K; a layer whose K is not a multiple of 64 is padded by prepare_layer to a multiple of
lcm(group, 64) with zero groups, which leaves every output unchanged.

The reference quantizer takes any group (quant/pack.py:6-23; its own test uses g16,
tests/test_svd_linear_cpu.py:10) and the group size is per-layer checkpoint metadata
(scripts/convert_simulated.py:209-214).  Bars as for the tuned path: activation codes (packed, and
the int8 operand) and scales bit-exact against the oracle quantizer; layer outputs within 1e-4
(float32 out) / 1e-3 (bf16 out) of the float64 evaluation, for W4A4 and W4A16, with LoRA.
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim, synth
from tests.gpu_util import (bf16_bits_of, bf16_tensor, device_adapters, operand_bytes, rel_l2, sx_pairs_ok,
                            to_device_state)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k,g", [(1, 64, 16), (77, 448, 32), (130, 1024, 16), (64, 1536, 32), (300, 768, 192),
                                   (33, 6144, 32)])
def test_any_group_codes_bit_exact(dev, m, k, g):
    from krea2_svdquant_amd.kernels.hip import backend, ops
    x = synth.make_activation(m, k, seed=m + g)
    st = synth.make_layer(64, k, x, rank=32, group_size=g, seed=4)
    prep = backend.prepare_layer(to_device_state(st, dev), (), dev)
    xd = bf16_tensor(x, dev)
    qa, sx, qx, xh, mid = ops.act_quant(xd, prep.srs, prep.l2, None, None, g, prep.rtp, ops.OPERAND_I8, True,
                                        True, False, False)
    qa2, sxp, _, _, _ = ops.act_quant(xd, prep.srs, prep.l2, None, None, g, prep.rtp, ops.OPERAND_I8, False, True,
                                      False, True)
    x_hat, packed, sx_ref, codes = sim.quantize_activations(x, st)
    assert np.array_equal(qx.cpu().numpy(), packed)
    assert np.array_equal(bf16_bits_of(sx), nm.bf16_bits(sx_ref))
    assert np.array_equal(bf16_bits_of(xh), nm.bf16_bits(x_hat))
    assert np.array_equal(qa.cpu().numpy(), operand_bytes(codes, "i8"))
    assert torch.equal(qa, qa2) and sx_pairs_ok(sxp, sx_ref)
    ref_mid = x_hat.astype(np.float64) @ st.l2.astype(np.float64).T
    assert rel_l2(ops.mid_values(mid).double().cpu().numpy()[:, :32], ref_mid) < 1e-5


@pytest.mark.parametrize("m,n,k,g,rl,bias", [
    (96, 256, 512, 32, 0, True),
    (200, 333, 1024, 16, 64, False),    # N % 8 != 0, LoRA
    (130, 384, 1536, 192, 32, True),    # a group spans three 64-column stages
    (257, 128, 6144, 32, 0, False),     # partial tiles, long K
    (50, 96, 80, 16, 0, True),          # K % 64 != 0: prepare_layer pads K to 128 (lcm(16, 64))
    (33, 160, 96, 32, 16, False),       # K = 96 -> 128, with LoRA
    (20, 64, 144, 48, 0, False),        # K = 144 -> 192 (lcm(48, 64))
])
@pytest.mark.parametrize("mode", ["w4a4", "w4a16"])
def test_any_group_layer_matches_oracle(dev, m, n, k, g, rl, bias, mode):
    from krea2_svdquant_amd.kernels.hip import backend
    x = synth.make_activation(m, k, seed=11 + g)
    st = synth.make_layer(n, k, x, rank=32, group_size=g, seed=12, bias=bias)
    if rl:
        st.adapters.append(synth.make_adapter(n, k, rank=rl, seed=13))
    prep = backend.prepare_layer(to_device_state(st, dev), device_adapters(st, dev), dev)
    ref = (sim.w4a4_eval if mode == "w4a4" else sim.w4a16_eval)(x, st)["y"]
    xd = bf16_tensor(x, dev)
    y32 = backend.forward_prepared(xd, prep, mode=mode, out_f32=True).cpu().numpy()
    y16 = backend.forward_prepared(xd, prep, mode=mode).float().cpu().numpy()
    e32, e16 = rel_l2(y32, ref), rel_l2(y16, nm.bf16(ref.astype(np.float32)))
    print(f"  g{g} {mode} M={m} N={n} K={k}: rel_l2 f32 {e32:.3e}, bf16 {e16:.3e}")
    assert e32 < 1e-4 and e16 < 1e-3


def test_g32_module_through_the_reference_api(dev):
    """A g32 checkpoint state through SVDQuantLinear (backend auto) with a LoRA adapter."""
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    x = synth.make_activation(80, 1024, seed=31)
    st = synth.make_layer(384, 1024, x, rank=32, group_size=32, seed=32, bias=True)
    mod = SVDQuantLinear(to_device_state(st, dev), backend="auto")
    ad = synth.make_adapter(384, 1024, rank=16, seed=33, scale=0.8)
    mod.add_lora_adapter(bf16_tensor(ad.down, dev), bf16_tensor(ad.up, dev), scale=0.8)
    st.adapters.append(ad)
    y = mod(bf16_tensor(x, dev)).float().cpu().numpy()
    assert rel_l2(y, nm.bf16(sim.w4a4_eval(x, st)["y"].astype(np.float32))) < 1e-3
