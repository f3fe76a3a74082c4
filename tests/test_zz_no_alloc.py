"""svdq_act_quant_noalloc (split partials in the library's device scratch) against svdq_act_quant
(caller workspace), through the C-ABI: two calls in a row, the second with a smaller input, every
output bit-identical (same kernels, same split count, same summation order), the codes bit-exact
against the oracle quantizer, and the W4A4 GEMM fed from the no-allocation head equal to the one
fed from the workspace head."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import sim, synth
from tests.gpu_util import bf16_tensor, e3m2_codes_of, sx_pairs_ok, to_device_state

pytestmark = pytest.mark.gpu


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _call_pair(dev, x, prep, st, g):
    from krea2_svdquant_amd.kernels.hip import lib, ops
    m, k = x.shape
    rtp = prep.rtp
    flags = lib.SVDQ_ACT_OPERAND_E3M2 | lib.SVDQ_ACT_SX_PAIRS
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    splits, mid_n = ctypes.c_int(), ctypes.c_int64()
    lib.call("svdq_act_quant_workspace", m, k, g, rtp, ctypes.byref(splits), ctypes.byref(mid_n))
    assert splits.value * m * rtp <= lib.SVDQ_ACT_NOALLOC_MAX_FLOATS
    rl = 0 if prep.lora_down is None else prep.lora_down.shape[0]
    lora = (None, 0, None) if rl == 0 else (_vp(prep.lora_down), rl, _vp(prep.lora_mult))
    outs = []
    for noalloc in (False, True):
        qa = torch.empty(ops.operand_bytes(m, k, ops.OPERAND_E3M2), dtype=torch.uint8, device=dev)
        sx = torch.empty((k // g, m), dtype=torch.int32, device=dev)
        if noalloc:
            mid = torch.full((1, m, rtp), float("nan"), dtype=torch.float32, device=dev)   # the head only
            lib.call("svdq_act_quant_noalloc", _vp(x), k, _vp(prep.srs), _vp(prep.l2), prep.l2.shape[0], lora[0],
                     lora[1], lora[2], m, k, g, rtp, flags, _vp(qa), _vp(sx), None, None, k, _vp(mid), stream)
        else:
            mid = torch.empty(mid_n.value, dtype=torch.float32, device=dev).view(splits.value + 1, m, rtp)
            lib.call("svdq_act_quant", _vp(x), k, _vp(prep.srs), _vp(prep.l2), prep.l2.shape[0], lora[0], lora[1],
                     lora[2], m, k, g, rtp, flags, _vp(qa), _vp(sx), None, None, k, _vp(mid), splits.value, stream)
        outs.append((qa, sx, mid[:1].clone()))
    torch.cuda.synchronize()
    (qa0, sx0, mid0), (qa1, sx1, mid1) = outs
    assert torch.equal(qa0, qa1) and torch.equal(sx0, sx1)
    assert torch.equal(mid0.view(torch.int32), mid1.view(torch.int32)), "finalized low-rank operand differs"
    _, _, sx_ref, codes = sim.quantize_activations(x.float().cpu().numpy(), st)
    assert np.array_equal(e3m2_codes_of(qa1.cpu().numpy(), m, k), codes)
    assert sx_pairs_ok(sx1, sx_ref)
    y = []
    for qa, sx, mid in outs:
        y.append(ops.w4a4_gemm(qa, sx, prep.weight_operand(ops.OPERAND_E3M2),
                               prep.weight_scale_pairs(ops.OPERAND_E3M2), mid, prep.l1cat, prep.bias, g,
                               ops.OPERAND_E3M2, True))
    assert torch.equal(y[0], y[1])
    return y[1]


def test_noalloc_matches_workspace_entry_point_twice_then_smaller(dev):
    from krea2_svdquant_amd.kernels.hip import backend
    k, n = 1536, 384
    xs = synth.make_activation(700, k, seed=61)
    st = synth.make_layer(n, k, xs, rank=32, group_size=64, seed=62, bias=True)
    st.adapters.append(synth.make_adapter(n, k, rank=16, seed=63))
    from tests.gpu_util import device_adapters
    prep = backend.prepare_layer(to_device_state(st, dev), device_adapters(st, dev), dev)
    # first call: 700 rows; second call, right after, with fewer rows (the scratch keeps the first
    # call's larger partials beyond what the second call writes)
    for m in (700, 130):
        x = bf16_tensor(xs[:m], dev)
        y = _call_pair(dev, x, prep, st, 64)
        ref = sim.w4a4_eval(xs[:m], st)["y"]
        e = sim.rel_l2(y.cpu().numpy(), ref)
        print(f"  noalloc M={m}: rel_l2 f32-out vs oracle {e:.3e}")
        assert e < 1e-4


def test_noalloc_config1_ffup_rows(dev):
    """The benchmark layer size (M=4096, K=6144, rank 32): the activation pass's K splits of 4096 x 32
    f32 partials (7 at this size, 3.5 MiB) in the file-scope array."""
    from krea2_svdquant_amd.kernels.hip import backend
    x = synth.make_activation(4096, 6144, seed=71)
    st = synth.make_layer(512, 6144, x[:256], rank=32, group_size=64, seed=72)
    prep = backend.prepare_layer(to_device_state(st, dev), (), dev)
    _call_pair(dev, bf16_tensor(x, dev), prep, st, 64)
