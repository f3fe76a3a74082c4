"""CPU checks of the test-side e3m2 (FP6) operand encoder the GPU parity tests compare against.

The encoder follows the OCP FP6 e3m2 definition (sign, 3 exponent bits with bias 3, 2 mantissa
bits; no infinities or NaNs); these checks pin it against the format's closed-form values and
the bit layout, so a wrong bias, field order or plane split fails here, not only on the GPU.
"""
import numpy as np

from tests.gpu_util import e3m2_code, e3m2_planar, e3m2_rows, e3m2_value


def test_e3m2_codes_are_exact_for_every_int4_code():
    q = np.arange(-8, 8)
    c = e3m2_code(q)
    assert np.array_equal(e3m2_value(c), q)              # every INT4 code is exact in e3m2
    assert c[q.tolist().index(1)] == 0b0_011_00           # 1.0 = 2^0: exponent field = bias
    assert c[q.tolist().index(-8)] == 0b1_110_00          # -8 = -2^3
    assert c[q.tolist().index(7)] == 0b0_101_11           # 7 = 1.75 * 2^2
    assert c[q.tolist().index(0)] == 0


def test_e3m2_decoder_covers_the_format():
    v = e3m2_value(np.arange(64))
    assert v.max() == 28.0 and v.min() == -28.0           # largest normal 1.75 * 2^4
    assert e3m2_value(np.array([1]))[0] == 0.0625         # smallest subnormal 2^-2 / 4
    assert len(set(np.abs(v).tolist())) == 32


def test_e3m2_planar_layout_fields_and_planes():
    rng = np.random.default_rng(0)
    r, k = 5, 192
    q = rng.integers(-8, 8, size=(r, k))
    buf = e3m2_planar(q)
    rp = 6
    assert buf.size == rp * k * 3 // 4
    rows = e3m2_rows(buf, r, k)                            # [K/64, 2, R, 24]
    for t in range(k // 64):
        for h in range(2):
            for row in range(r):
                v = int.from_bytes(rows[t, h, row].tobytes(), "little")
                fields = [(v >> (6 * f)) & 63 for f in range(32)]
                assert np.array_equal(e3m2_value(np.array(fields)), q[row, 64 * t + 32 * h:64 * t + 32 * h + 32])
    # padding row of the Q planes is zero and sits between row r - 1 and the next plane
    qpl = buf[:(k // 64) * 2 * rp * 16].reshape(k // 64, 2, rp, 16)
    assert not qpl[:, :, r:].any()
