"""GPU parity for ranks beyond one launch of the activation pass, and the module's operand cache.

The down projections run in launches of 4 MFMA column tiles of 32 (rank r in ceil(r/32) tiles, then
the concatenated LoRA ranks): r = 64 with two rank-64 adapters (the reference's MLP rank with two
adapters, 6 tiles) and r = 160 with a rank-48 adapter (the low-rank tiles themselves span both
launches).  Padded ranks up to 256 take the GEMM's low-rank term in 32-rank LDS chunks; r = 32 with
adapters of ranks 128, 128 and 40 (padded rank 352) takes its global-memory path.  Reference: runtime/linear.py:88-111,156-161 (any number of adapters, each on the raw x).
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim, synth
from tests.gpu_util import bf16_tensor, device_adapters, rel_l2, to_device_state

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("r,ranks,mode,n", [
    (64, (64, 64), "w4a4", 384), (64, (64, 64), "w4a16", 384),
    (160, (48,), "w4a4", 384), (32, (128, 16, 40), "w4a4", 384), (32, (128, 128, 40), "w4a4", 384),
    (32, (128, 16), "w4a4", 200),   # padded rank 192 in LDS chunks, a partial column tile
])
def test_many_tiles_match_oracle(dev, r, ranks, mode, n):
    from krea2_svdquant_amd.kernels.hip import backend, ops
    m, k = 300, 1024
    x = synth.make_activation(m, k, seed=81)
    st = synth.make_layer(n, k, x, rank=r, group_size=64, seed=82, bias=True)
    for i, rl in enumerate(ranks):
        st.adapters.append(synth.make_adapter(n, k, rank=rl, seed=83 + i, scale=0.5 + 0.25 * i))
    prep = backend.prepare_layer(to_device_state(st, dev), device_adapters(st, dev), dev)
    tiles = -(-r // 32) + -(-sum(ranks) // 32)
    assert tiles > 4 and prep.rtp >= r + sum(ranks)
    xd = bf16_tensor(x, dev)
    # the down projections at the workspace head, every column
    opc = ops.OPERAND_E3M2 if mode == "w4a4" else ops.OPERAND_NONE
    out = ops.act_quant(xd, prep.srs, prep.l2, prep.lora_down, prep.lora_mult, 64, prep.rtp, opc, False,
                        mode == "w4a16", False, mode == "w4a4")
    got = ops.mid_values(out[4]).double().cpu().numpy()
    ref = sim.w4a4_eval(x, st)
    expect = np.zeros((m, prep.rtp))
    expect[:, :r] = ref["mid"]
    col = r
    for ad in st.adapters:
        expect[:, col:col + ad.rank] = ad.multiplier * (x.astype(np.float64) @ nm.bf16(ad.down).astype(np.float64).T)
        col += ad.rank
    assert rel_l2(got, expect) < 1e-5
    assert (got[:, col:] == 0).all()
    # the layer
    evaluate = sim.w4a4_eval if mode == "w4a4" else sim.w4a16_eval
    y_ref = evaluate(x, st)["y"]
    y32 = backend.forward_prepared(xd, prep, mode=mode, out_f32=True).cpu().numpy()
    y16 = backend.forward_prepared(xd, prep, mode=mode).float().cpu().numpy()
    e32, e16 = rel_l2(y32, y_ref), rel_l2(y16, nm.bf16(y_ref.astype(np.float32)))
    print(f"  r={r} LoRA ranks {ranks} ({tiles} tiles, {mode}): rel_l2 f32 {e32:.3e}, bf16 {e16:.3e}")
    assert e32 < 1e-4 and e16 < 1e-3


def test_module_cache_follows_adapter_changes_and_shares_the_weight_operand(dev):
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    m, n, k = 96, 256, 512
    x = synth.make_activation(m, k, seed=91)
    st = synth.make_layer(n, k, x, rank=64, group_size=64, seed=92)
    mod = SVDQuantLinear(to_device_state(st, dev), backend="hip_gfx950")
    ad = synth.make_adapter(n, k, rank=64, seed=93, scale=0.8)
    mod.add_lora_adapter(bf16_tensor(ad.down, dev), bf16_tensor(ad.up, dev), scale=0.8)
    st.adapters.append(ad)
    xd = bf16_tensor(x, dev)

    def check():
        y = mod(xd).float().cpu().numpy()
        e = rel_l2(y, nm.bf16(sim.w4a4_eval(x, st)["y"].astype(np.float32)))
        assert e < 1e-3, e

    check()
    # the multiplier is read on every forward (reference linear.py:42-45)
    mod.lora_adapters[0].scale = 0.3
    st.adapters[0] = sim.Adapter(ad.down, ad.up, scale=0.3)
    check()
    # an in-place edit of an adapter weight is picked up
    with torch.no_grad():
        mod.lora_adapters[0].up_weight.mul_(2)
    st.adapters[0] = sim.Adapter(ad.down, nm.bf16(ad.up * 2), scale=0.3)
    check()
    # _forward_base and forward share one expanded weight operand and its scale pairs
    base = mod._prepared[False][1]
    full = mod._prepared[True][1]
    assert base.operands and full.operands is base.operands and full.scale_pairs is base.scale_pairs
    mod._forward_base(xd)
    assert len(base.operands) == 1
