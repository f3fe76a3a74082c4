"""GPU parity of the gfx950 kernels against the CPU oracle (through the C-ABI custom ops).

Bars: activation codes, scales and x_hat bit-exact; GEMM / layer outputs within
relative L2 1e-3 of the float64 evaluation of the same quantized math -- in float32-output mode
directly, in bf16-output mode against bf16(oracle) (a bf16 store alone costs ~1.7e-3 against
float32, so the bf16 output is compared with the rounded reference).  Float32 mode is also
held to 1e-4, the bound the exact integer group sums allow.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import pack as op
from oracle import sim, synth
from tests.gpu_util import (bf16_bits_of, bf16_tensor, device_adapters, e3m2_planar, e3m2_rows, operand_bytes,
                            rel_l2, to_device_state)
from tests.golden_io import load_layer_fixture

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
TOL, TOL_F32 = 1e-3, 1e-4


def _ops():
    from krea2_svdquant_amd.kernels.hip import backend, ops
    return backend, ops


def _run_act(x_np, st, dev, operand="e4m3", packed=True, xhat=False, exact=False, adapters=True, sx_pairs=False):
    """Returns (qa, sx, qx, xhat, mid) from svdq::act_quant."""
    backend, ops = _ops()
    prep = backend.prepare_layer(to_device_state(st, dev), device_adapters(st, dev) if adapters else (), dev)
    x = bf16_tensor(x_np, dev)
    opc = ops.OPERAND_NONE if operand is None else ops.OPERAND_NAMES[operand]
    out = ops.act_quant(x, prep.srs, prep.l2, prep.lora_down, prep.lora_mult, st.group_size, prep.rtp,
                        opc, packed, xhat, exact, sx_pairs)
    torch.cuda.synchronize()
    return out, prep


def test_w4a4_gemm_layout_identity(dev):
    """qx = identity codes -> y must equal the weight codes transposed (MFMA D layout check)."""
    _, ops = _ops()
    m, k, n = 64, 64, 128
    q = np.zeros((m, k), np.int8)
    q[np.arange(m), np.arange(m)] = 1
    qw = ((np.arange(n)[:, None] * 7 + np.arange(k)[None, :] * 3) % 15 - 7).astype(np.int8)
    sx = torch.full((1, m), 0x3F803F80, dtype=torch.int32, device=dev)   # bf16 pair (1.0, 1.0), [K/G, M]
    qwt = torch.from_numpy(op.pack_int4(qw)).to(dev)
    sw = torch.ones((n, 1), dtype=torch.float16, device=dev)
    mid = torch.zeros((1, m, 32), dtype=torch.float32, device=dev)
    l1 = torch.zeros((n, 32), dtype=torch.bfloat16, device=dev)
    expect = qw[:, :m].T.astype(np.float32)
    for fmt in ("e4m3", "i8", "e3m2"):
        qa = torch.from_numpy(e3m2_planar(q) if fmt == "e3m2" else operand_bytes(q, fmt)).to(dev)
        opc = ops.OPERAND_NAMES[fmt]
        y = ops.w4a4_gemm(qa, sx, ops.prepare_weight_operand(qwt, opc), ops.prepare_weight_scales(sw, opc), mid, l1,
                          None, 64, opc, True).cpu().numpy()
        if not np.array_equal(y, expect):
            bad = np.argwhere(y != expect)
            rows = {int(r): [int(rr) for rr in np.where((expect == y[r]).all(1))[0]] for r in range(m)}
            pytest.fail(f"{fmt}: {len(bad)} mismatches, first {bad[:4].tolist()}; row matches {rows}")


@pytest.mark.parametrize("fmt", ["e4m3", "i8", "e3m2"])
@pytest.mark.parametrize("n", [300, 301])
def test_weight_operand_matches_unpacked_codes(dev, fmt, n):
    """The per-layer expanded weight operand holds exactly the oracle's unpacked codes."""
    _, ops = _ops()
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, size=(n, 448), dtype=np.uint8)   # every nibble value, K = 896
    out = ops.prepare_weight_operand(torch.from_numpy(packed).to(dev), ops.OPERAND_NAMES[fmt]).cpu().numpy()
    codes = op.unpack_int4(packed)
    if fmt == "e3m2":
        assert out.size == ((n + 1) & ~1) * 896 * 3 // 4
        assert np.array_equal(e3m2_rows(out, n, 896), e3m2_rows(e3m2_planar(codes), n, 896))
    else:
        assert np.array_equal(out, operand_bytes(codes, fmt))


@pytest.mark.parametrize("name", ["w4a4_small_g64.npz", "w4a4_small_g128.npz"])
def test_act_quant_golden_bit_exact(dev, name):
    fx, x, st = load_layer_fixture(GOLDEN / name)
    (qa, sx, qx, xh, mid), _ = _run_act(x, st, dev, operand="e4m3", packed=True, xhat=True)
    assert np.array_equal(qx.cpu().numpy(), fx["qx_packed"])
    assert np.array_equal(bf16_bits_of(sx), fx["sx"])
    assert np.array_equal(bf16_bits_of(xh), fx["xhat"])
    codes = op.unpack_int4(fx["qx_packed"])
    assert np.array_equal(qa.cpu().numpy(), operand_bytes(codes, "e4m3"))
    (_, sxp, _, _, _), _ = _run_act(x, st, dev, operand="e4m3", packed=False, sx_pairs=True)
    bits = fx["sx"].astype(np.uint32)
    assert np.array_equal(sxp.cpu().numpy().view(np.uint32), (bits | (bits << 16)).T)
    (qa8, sx8, qx8, _, _), _ = _run_act(x, st, dev, operand="i8", packed=True)
    assert np.array_equal(qa8.cpu().numpy(), operand_bytes(codes, "i8"))
    (qa6, sx6, _, _, _), _ = _run_act(x, st, dev, operand="e3m2", packed=False, sx_pairs=True)
    m, k = codes.shape
    assert np.array_equal(e3m2_rows(qa6.cpu().numpy(), m, k), e3m2_rows(e3m2_planar(codes), m, k))
    assert np.array_equal(sx6.cpu().numpy().view(np.uint32), (bits | (bits << 16)).T)
    assert np.array_equal(qx8.cpu().numpy(), fx["qx_packed"]) and np.array_equal(bf16_bits_of(sx8), fx["sx"])
    (_, _, _, xh16, _), _ = _run_act(x, st, dev, operand=None, packed=False, xhat=True)
    assert np.array_equal(bf16_bits_of(xh16), fx["xhat"])
    r = st.l2.shape[0]
    ad = st.adapters[0]
    lmid = ad.multiplier * (x.astype(np.float64) @ ad.down.astype(np.float64).T)
    _, ops = _ops()
    got = ops.mid_values(mid).double().cpu().numpy()
    assert rel_l2(got[:, :r], fx["mid"]) < 1e-5
    assert rel_l2(got[:, r:r + ad.rank], lmid) < 1e-5
    assert (got[:, r + ad.rank:] == 0).all()


def test_act_quant_edge_rows_bit_exact(dev):
    fx = np.load(GOLDEN / "edge_activations.npz")
    x = nm.from_bf16_bits(fx["x"])
    k = x.shape[1]
    st = sim.LayerState(smooth=nm.from_bf16_bits(fx["smooth"]), qweight=np.full((32, k // 2), 0x88, np.uint8),
                        weight_scales=np.ones((32, k // 64), np.float32), l1=np.zeros((32, 32), np.float32),
                        l2=np.zeros((32, k), np.float32), bias=None, group_size=64, shape=(32, k))
    codes = op.unpack_int4(fx["qx_packed"])
    for exact in (False, True):
        (qa, sx, qx, xh, _), _ = _run_act(x, st, dev, packed=True, xhat=True, exact=exact)
        assert np.array_equal(qx.cpu().numpy(), fx["qx_packed"]), f"exact={exact}"
        assert np.array_equal(bf16_bits_of(sx), fx["sx"]), f"exact={exact}"
        assert np.array_equal(bf16_bits_of(xh), fx["xhat"]), f"exact={exact}"
        assert np.array_equal(qa.cpu().numpy(), operand_bytes(codes, "e4m3")), f"exact={exact}"
        (qa2, sx2, qx2, _, _), _ = _run_act(x, st, dev, packed=True, xhat=False, exact=exact)
        assert np.array_equal(qx2.cpu().numpy(), fx["qx_packed"]) and np.array_equal(bf16_bits_of(sx2), fx["sx"])
        assert np.array_equal(qa2.cpu().numpy(), operand_bytes(codes, "e4m3"))


@pytest.mark.parametrize("m,k,g", [(1, 64, 64), (5, 448, 64), (64, 1024, 64), (100, 768, 128), (257, 1536, 64),
                                   (600, 6144, 64)])
def test_act_quant_random_shapes_bit_exact(dev, m, k, g):
    x = synth.make_activation(m, k, seed=m + k)
    st = synth.make_layer(64, k, x, rank=32, group_size=g, seed=3)
    (qa, sx, qx, _, mid), _ = _run_act(x, st, dev, adapters=False)
    xh, packed, sxo, codes = sim.quantize_activations(x, st)
    assert np.array_equal(qx.cpu().numpy(), packed)
    assert np.array_equal(qa.cpu().numpy(), operand_bytes(codes, "e4m3"))
    assert np.array_equal(bf16_bits_of(sx), nm.bf16_bits(sxo))
    ref_mid = xh.astype(np.float64) @ st.l2.astype(np.float64).T
    _, ops = _ops()
    assert rel_l2(ops.mid_values(mid).double().cpu().numpy()[:, :32], ref_mid) < 1e-5
    _check_mid_head(mid)


def _check_mid_head(mid):
    """The workspace head is the split partials summed in split order (float32), then split into
    bf16 hi = bf16(v) and lo = bf16(v - hi): bit for bit."""
    part = mid[1:].float()
    v = part[0].clone()
    for s in range(1, part.shape[0]):
        v = v + part[s]
    hi = v.to(torch.bfloat16)
    lo = (v - hi.float()).to(torch.bfloat16)
    m, rtp = v.shape
    planes = mid[0].contiguous().view(torch.bfloat16).view(m, 2, rtp)
    assert torch.equal(planes[:, 0].view(torch.int16), hi.view(torch.int16))
    assert torch.equal(planes[:, 1].view(torch.int16), lo.view(torch.int16))


def _layer_outputs(x_np, st, dev, mode, out_f32, operand="e4m3"):
    backend, _ = _ops()
    prep = backend.prepare_layer(to_device_state(st, dev), device_adapters(st, dev), dev)
    y = backend.forward_prepared(bf16_tensor(x_np, dev), prep, mode=mode, out_f32=out_f32, operand=operand)
    return y.float().cpu().numpy()


def _check_layer(x, st, dev, mode, ref):
    for operand in (("e4m3", "i8", "e3m2") if mode == "w4a4" else ("e4m3",)):
        y32 = _layer_outputs(x, st, dev, mode, True, operand)
        e32 = rel_l2(y32, ref)
        y16 = _layer_outputs(x, st, dev, mode, False, operand)
        e16 = rel_l2(y16, nm.bf16(ref.astype(np.float32)))
        print(f"  {mode}/{operand}: rel_l2 f32-out={e32:.3e} bf16-out vs bf16(ref)={e16:.3e}")
        assert e32 < TOL_F32 and e16 < TOL


@pytest.mark.parametrize("name", ["w4a4_small_g64.npz", "w4a4_small_g128.npz"])
@pytest.mark.parametrize("mode", ["w4a4", "w4a16"])
def test_layer_golden(dev, name, mode):
    fx, x, st = load_layer_fixture(GOLDEN / name)
    _check_layer(x, st, dev, mode, fx["y_" + mode])


@pytest.mark.parametrize("m,n,k,g,r,rl,bias", [
    (128, 128, 64, 64, 32, 0, False),     # one group: a single, half-filled pipeline stage
    (200, 333, 640, 64, 32, 64, True),
    (7, 1536, 2048, 64, 64, 0, True),
    (256, 512, 6144, 64, 32, 64, False),
    (130, 200, 448, 64, 32, 0, True),     # 7 groups: 4 stages, the last one a single group
    (64, 256, 1152, 64, 32, 32, False),   # 18 groups: 9 stages
    (96, 320, 384, 128, 32, 0, True),     # group 128: 3 stages
    (33, 128, 896, 128, 64, 64, False),   # group 128: 7 stages
    (70, 100, 256, 64, 32, 0, True),      # two stages; N % 8 != 0 (element stores at the tile edge)
    (50, 136, 128, 128, 32, 32, False),   # group 128: a single stage
    # K a multiple of 512: the e3m2 kernel's paired-stage main loop (the others take its
    # general loop); rank 32 without LoRA puts the epilogue operands in LDS
    (300, 264, 512, 64, 32, 0, True),     # two stages: only the peeled pair
    (130, 200, 1536, 64, 32, 0, False),   # six stages
    (96, 384, 1024, 128, 32, 0, True),    # group 128, four stages
    (64, 130, 2560, 128, 32, 16, True),   # group 128, ten stages, LoRA
])
@pytest.mark.parametrize("mode", ["w4a4", "w4a16"])
def test_layer_random_shapes(dev, m, n, k, g, r, rl, bias, mode):
    x = synth.make_activation(m, k, seed=11)
    st = synth.make_layer(n, k, x, rank=r, group_size=g, seed=12, bias=bias)
    if rl:
        st.adapters.append(synth.make_adapter(n, k, rank=rl, seed=13))
    ref = (sim.w4a4_eval if mode == "w4a4" else sim.w4a16_eval)(x, st)["y"]
    _check_layer(x, st, dev, mode, ref)


@pytest.mark.parametrize("m,n,k,g,bias", [
    # the one-wave-per-SIMD W4A16 kernel; tile height 192 where it needs no more rounds of tiles
    # over the 256 CUs than 256 does, else 256
    (2304, 4096, 512, 64, False),    # 192 tiles of 192 x 256
    (2100, 4300, 576, 64, True),     # 192-row tiles, partial last tiles in M and N; 9 stages (odd: the tail stage)
    (2048, 4352, 640, 128, False),   # group 128, 192-row tiles
    (4096, 4096, 512, 64, True),     # 256 tiles of 256 x 256 (192-row tiles would need 2 rounds)
    (2304, 16384, 384, 64, False),   # config 2 ff.up's tiling at short K: 768 tiles of 192 x 256
])
def test_w4a16_wide_tiles(dev, m, n, k, g, bias):
    x = synth.make_activation(m, k, seed=17)
    st = synth.make_layer(n, k, x, rank=32, group_size=g, seed=18, bias=bias)
    _check_layer(x, st, dev, "w4a16", sim.w4a16_eval(x, st)["y"])


def test_outputs_deterministic(dev):
    x = synth.make_activation(300, 2048, seed=21)
    st = synth.make_layer(640, 2048, x, rank=32, group_size=64, seed=22, bias=True)
    st.adapters.append(synth.make_adapter(640, 2048, rank=64, seed=23))
    a = _layer_outputs(x, st, dev, "w4a4", True)
    b = _layer_outputs(x, st, dev, "w4a4", True)
    assert np.array_equal(a, b)
