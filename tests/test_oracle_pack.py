"""Pins the oracle's INT4 quantizer / packing (oracle/pack.py) without retyping its formulas.

Checks used:
* the reference's own known-answer test (tests/test_pack.py:6-10: all 16 codes round trip)
  and shape test (:13-18: K=130, g64 pads to 192), via committed golden data;
* explicit byte values of the nibble layout;
* torch's native bf16 / fp16 arithmetic applied the way the reference applies it
  (an independent implementation of the rounding the numpy oracle emulates bit by bit);
* brute force: every code is the integer in [-8, 7] nearest to x / scale, ties to even;
* closed forms: all-zero group, exact .5 ties, the group maximum maps to +-7.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import pack as op

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_reference_known_answer_pack_roundtrip():
    ka = json.loads((GOLDEN / "reference_known_answers.json").read_text())
    q = np.array(ka["pack_roundtrip"]["codes"], dtype=np.int8)
    packed = op.pack_int4(q)
    assert packed.tolist() == ka["pack_roundtrip"]["packed"]
    assert np.array_equal(op.unpack_int4(packed, q.shape[-1]), q)


def test_nibble_layout_bytes():
    assert op.pack_int4(np.array([[-8, 7]], np.int8)).tolist() == [[0xF0]]
    assert op.pack_int4(np.array([[7, -8]], np.int8)).tolist() == [[0x0F]]
    assert op.pack_int4(np.array([[0, 0]], np.int8)).tolist() == [[0x88]]
    assert op.pack_int4(np.array([[1, -1, 3]], np.int8)).tolist() == [[0x79, 0x8B]]  # odd K padded with 0
    assert op.unpack_int4(np.array([[0x00, 0xFF]], np.uint8)).tolist() == [[-8, -8, 7, 7]]


def test_reference_shape_case_pads_to_group():
    x = np.random.default_rng(0).standard_normal((7, 130)).astype(np.float32)
    q, s = op.quantize_symmetric_int4(x, 64, "f32")
    y = op.dequantize_symmetric_int4(q, s, 64, "f32")
    assert q.shape == (7, 192) and s.shape == (7, 3) and y.shape[-1] == 192
    assert np.isfinite(y).all() and (q[:, 130:] == 0).all()


def _torch_quant_like_reference(x: torch.Tensor, g: int):
    """The reference's torch call sequence (quant/pack.py:17-21), run by torch itself."""
    grouped = x.reshape(x.shape[0], -1, g)
    scales = grouped.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 7.0
    q = torch.round(grouped.float() / scales).clamp(-8, 7).to(torch.int8)
    return q.reshape(x.shape), scales.squeeze(-1)


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float32, "f32"), (torch.float16, "fp16")])
def test_quantizer_matches_torch_arithmetic(dtype, name):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((33, 256)).astype(np.float32) * 3
    x[:, 5] *= 40
    if dtype != torch.float16:      # fp16 cannot hold the 1e-8 floor: 0/0 in the reference too
        x[3] = 0.0                  # all-zero groups
        x[4, :64] = 1e-30           # tiny group
    xt = torch.from_numpy(x).to(dtype)
    q_ref, s_ref = _torch_quant_like_reference(xt, 64)
    q, s = op.quantize_symmetric_int4(xt.float().numpy(), 64, name)
    assert np.array_equal(q, q_ref.numpy())
    assert np.array_equal(s, s_ref.float().numpy())


def test_codes_are_nearest_integer_ties_to_even_bruteforce():
    rng = np.random.default_rng(2)
    x = nm.bf16(rng.standard_normal((8, 128)).astype(np.float32))
    q, s = op.quantize_symmetric_int4(x, 64, "bf16")
    ratio = (x.reshape(8, 2, 64) / s[..., None]).astype(np.float32)   # float32 division, as torch
    cand = np.arange(-8, 8)
    for idx in np.ndindex(ratio.shape):
        d = np.abs(ratio[idx] - cand)
        best = cand[d == d.min()]
        expect = best[best % 2 == 0][0] if len(best) == 2 else best[0]
        assert q.reshape(8, 2, 64)[idx] == expect


def test_closed_forms_zero_group_ties_and_max():
    s_zero = float(nm.bf16(np.float32(nm.BF16_1E_8) / np.float32(7)))
    q, s = op.quantize_symmetric_int4(np.zeros((1, 64), np.float32), 64, "bf16")
    assert (q == 0).all() and s[0, 0] == np.float32(s_zero)
    # amax 7 -> scale exactly 1: x = 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, -0.5 -> 0, 7 -> 7
    row = np.zeros((1, 64), np.float32)
    row[0, :6] = [7.0, 2.5, 3.5, -2.5, -0.5, 1.5]
    q, s = op.quantize_symmetric_int4(row, 64, "bf16")
    assert s[0, 0] == 1.0 and q[0, :6].tolist() == [7, 2, 4, -2, 0, 2]
    assert op.quantize_symmetric_int4(-row, 64, "bf16")[0][0, :6].tolist() == [-7, -2, -4, 2, 0, -2]


def test_smoothing_matches_torch_bf16_division():
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((16, 512)).astype(np.float32) * 5).to(torch.bfloat16)
    s = torch.from_numpy(rng.uniform(0.2, 40.0, 512).astype(np.float32)).to(torch.bfloat16)
    ref = (x / s).float().numpy()
    got = op.smooth_activations(x.float().numpy(), s.float().numpy())
    assert np.array_equal(nm.bf16_bits(got), nm.bf16_bits(ref))


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float32, "f32")])
def test_dequantize_matches_torch_arithmetic(dtype, name):
    rng = np.random.default_rng(4)
    q = rng.integers(-8, 8, (12, 128)).astype(np.int8)
    sc = rng.uniform(1e-3, 2.0, (12, 2)).astype(np.float32)
    sc16 = torch.from_numpy(sc).to(torch.float16)
    ref = (torch.from_numpy(q).reshape(12, 2, 64).to(dtype) * sc16.to(dtype).unsqueeze(-1)).reshape(12, 128)
    got = op.dequantize_symmetric_int4(q, sc16.float().numpy(), 64, name)
    assert np.array_equal(got, ref.float().numpy())


def test_bf16_rounding_matches_torch_exhaustive_neighbourhood():
    rng = np.random.default_rng(5)
    f = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 65504.0, 1e-40], np.float32)])
    f = f.astype(np.float32)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(nm.bf16_bits(f), ref)
