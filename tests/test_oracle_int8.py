"""Pins of the oracle's MXINT8 weight quantizer (the bfloat8_b counterpart).

The oracle encodes by a nearest search over the candidate codes with explicit tie-breaking; these tests check it
against an independent route, numpy's round-half-to-even of 64 v clipped to [-128, 127] (the OCP Microscaling
specification's element rounding for MXINT8), over every bf16 value in range; the block scale against its
closed form 2^floor(log2 amax) computed with numpy's log2; the dequantized error against half a code step.
"""

import numpy as np
import pytest

import oracle


def np_code(v):
    return np.clip(np.round(np.asarray(v, np.float64) * 64.0), -128, 127).astype(np.int64)


def test_encode_every_bf16_value_against_numpy_rounding():
    bits = np.arange(0, 1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 4)]
    assert v.size > 30000
    got = np.array([oracle.mxint8_encode(x) for x in v])
    assert np.array_equal(got, np_code(v))


def test_encode_ties_and_saturation():
    # halfway between two codes goes to the even code; past 127/64 saturates; -2 is code -128
    assert [oracle.mxint8_encode(x) for x in (0.5 / 64, 1.5 / 64, 2.5 / 64, -0.5 / 64, -1.5 / 64)] == [0, 2, 2, 0, -2]
    assert [oracle.mxint8_encode(x) for x in (127.4 / 64, 127.5 / 64, 1.999, 2.0, 1e30)] == [127] * 5
    assert [oracle.mxint8_encode(x) for x in (-2.0, -128.5 / 64, -3.0, -1e30)] == [-128] * 4
    assert oracle.mxint8_encode(1.0) == 64 and oracle.mxint8_encode(-0.015625) == -1


@pytest.mark.parametrize("amax, code", [(1.0, 127), (1.999, 127), (2.0, 128), (0.75, 126), (0.0, 0),
                                        (2.0 ** -130, 0), (1e38, 253), (0.02, 121), (0.05, 122)])
def test_scale_code_closed_form(amax, code):
    assert oracle.mxint8_scale_code(amax) == code
    if amax > 2.0 ** -126:
        assert code == 127 + int(np.floor(np.log2(amax)))


def test_quantize_blocks_scale_and_error_bound():
    rng = np.random.default_rng(11)
    N, K = 9, 256
    w = (rng.standard_normal((N, K)) * np.exp2(rng.uniform(-10, 3, (N, K // 32))).repeat(32, axis=1)).astype(np.float32)
    w[0, :32] = 0.0       # an all-zero block
    w[1, 40] = -100.0     # a block dominated by one value
    w[2, 64] = 1.999 * 2.0 ** -3  # a block whose largest value saturates to code 127
    q, sc = oracle.quantize_mxint8(w)
    amax = np.abs(w.reshape(N, K // 32, 32)).max(2).astype(np.float64)
    ref = np.where(amax > 0, 127 + np.floor(np.log2(np.where(amax > 0, amax, 1))), 0).astype(np.int64)
    assert np.array_equal(sc.astype(np.int64), ref)
    assert sc[0, 0] == 0 and np.all(q[0, :32] == 0)
    deq = oracle.dequantize_mxint8(q, sc).astype(np.float64)
    step = np.ldexp(1.0, sc.astype(np.int32) - 133).repeat(32, axis=1)
    err = np.abs(deq - w)
    # half a step, except the values that saturate at 127 steps (within one step of 2 X)
    sat = q == 127
    assert np.all(err[~sat] <= 0.5 * step[~sat] + 1e-30)
    assert np.all(err[sat] <= step[sat])
    # the codes are numpy's rounding of w / step
    assert np.array_equal(q.astype(np.int64), np.clip(np.round(w / step), -128, 127).astype(np.int64))


def test_dequantized_weights_are_fixed_points():
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((16, 128)) * 0.02).astype(np.float32)
    q, sc = oracle.quantize_mxint8(w)
    deq = oracle.dequantize_mxint8(q, sc)
    q2, sc2 = oracle.quantize_mxint8(deq)
    assert np.array_equal(oracle.dequantize_mxint8(q2, sc2), deq)
    # every dequantized value is a bf16 value (the GPU path widens the codes to bf16 exactly)
    b = deq.view(np.uint32)
    assert np.all((b & 0xFFFF) == 0)


def test_relative_error_of_gaussian_weights():
    """The format's precision on N(0, 0.02) weights: about 7 significant bits under a shared exponent, the
    bfloat8_b class (the reference reports ~1.2% layer error in bfp8, wormhole_n150/qwen3.5_9B/README.md:35-36)."""
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((64, 4096)) * 0.02).astype(np.float32)
    q, sc = oracle.quantize_mxint8(w)
    rel = np.linalg.norm(oracle.dequantize_mxint8(q, sc) - w) / np.linalg.norm(w)
    assert 2e-3 < rel < 1e-2
