"""Pins of the oracle's MXFP4 weight quantizer (the 4-bit weight path).

The oracle encodes by exhaustive nearest search over the E2M1 magnitudes; these tests check it against an
independent route, the decision thresholds of nearest-even rounding on the E2M1 grid written out from the
OCP Microscaling specification, over every bf16 value in range; the block scale against its closed form
2^(floor(log2 amax) - 2); the dequantized error against the grid spacing.
"""

import numpy as np
import pytest

import oracle

GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def threshold_code(v):
    """E2M1 code by the midpoint thresholds of the grid: a midpoint goes to the even code (0, 2, 4, 6)."""
    a = abs(float(v))
    if a <= 0.25:
        c = 0
    elif a < 0.75:
        c = 1
    elif a <= 1.25:
        c = 2
    elif a < 1.75:
        c = 3
    elif a <= 2.5:
        c = 4
    elif a < 3.5:
        c = 5
    elif a <= 5.0:
        c = 6
    else:
        c = 7
    return c | (8 if np.signbit(v) else 0)


def test_decode_table_closed_form():
    t = oracle.e2m1_table()
    assert list(t[:8]) == GRID
    assert list(-t[8:]) == GRID and np.signbit(t[8])


def test_encode_every_bf16_value_against_thresholds():
    bits = np.arange(0, 1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 16)]
    assert v.size > 30000
    got = np.array([oracle.e2m1_encode(x) for x in v])
    want = np.array([threshold_code(x) for x in v])
    assert np.array_equal(got, want)


def test_encode_ties_and_saturation():
    # midpoints go to the even mantissa, values past 6 saturate
    assert [oracle.e2m1_encode(x) for x in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)] == [0, 2, 2, 4, 4, 6, 6]
    assert [oracle.e2m1_encode(x) for x in (6.0, 7.99, 1e30)] == [7, 7, 7]
    assert oracle.e2m1_encode(-6.5) == 15 and oracle.e2m1_encode(-0.1) == 8


@pytest.mark.parametrize("amax, code", [(1.0, 125), (6.0, 127), (4.0, 127), (3.99, 126), (8.0, 128), (0.0, 0),
                                        (2.0 ** -130, 0), (1e38, 251), (0.02, 119)])
def test_scale_code_closed_form(amax, code):
    assert oracle.mx_scale_code(amax) == code


def test_quantize_blocks_scale_and_error_bound():
    rng = np.random.default_rng(7)
    N, K = 9, 256
    w = (rng.standard_normal((N, K)) * np.exp2(rng.uniform(-10, 3, (N, K // 32))).repeat(32, axis=1)).astype(np.float32)
    w[0, :32] = 0.0       # an all-zero block
    w[1, 40] = -100.0     # a block dominated by one value
    q, sc = oracle.quantize_mxfp4(w)
    amax = np.abs(w.reshape(N, K // 32, 32)).max(2)
    X = np.ldexp(1.0, sc.astype(np.int32) - 127)
    ref = np.where(amax > 0, np.ldexp(1.0, np.floor(np.log2(np.where(amax > 0, amax, 1))).astype(int) - 2), 2.0 ** -127)
    assert np.array_equal(X, ref)
    assert sc[0, 0] == 0 and np.all(q[0, :32] == 0)
    deq = oracle.dequantize_mxfp4(q, sc)
    Xk = X.repeat(32, axis=1)
    r = np.abs(w) / Xk
    # spacing of the grid is 0.5 up to 2, 1 up to 4, 2 up to 6; past 6 the value saturates
    bound = np.where(r <= 2, 0.25, np.where(r <= 4, 0.5, np.where(r <= 6, 1.0, r - 6))) * Xk * (1 + 1e-6)
    assert np.all(np.abs(deq - w) <= bound)
    # the block maximum lands on 4 X or 6 X
    blockmax = np.abs(deq.reshape(N, K // 32, 32)).max(2)
    assert np.all((blockmax[amax > 0] == 4 * X[amax > 0]) | (blockmax[amax > 0] == 6 * X[amax > 0]))


def test_known_answer_unit_scale():
    """A block whose largest magnitude is 6 has scale 1 (code 127) and keeps grid values exactly."""
    vals = [6.0, -4.0, 0.5, 0.0, 1.5, -3.0, 2.0, -0.5] * 4
    q, sc = oracle.quantize_mxfp4(np.array([vals], np.float32))
    assert sc[0, 0] == 127
    assert list(q[0, :8]) == [7, 14, 1, 0, 3, 13, 4, 9]
    np.testing.assert_array_equal(oracle.dequantize_mxfp4(q, sc)[0], np.array(vals, np.float32))
