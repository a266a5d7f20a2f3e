"""Pins of the oracle's E4M3 weight quantizer (the low-precision weight path).

The E4M3 decode table and the nearest-even encoding are checked against torch.float8_e4m3fn, an independent
implementation of the same OCP format; the per-row scale and the error bound against their closed forms.
"""

import numpy as np
import pytest
import torch

import oracle


def torch_encode(v):
    """torch's float32 -> float8_e4m3fn (nearest, ties to even; NaN above 464) as codes."""
    return torch.from_numpy(np.asarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def encode(v):
    return np.array([oracle.e4m3_encode(x) for x in np.asarray(v, np.float32).ravel()], np.uint8)


def test_decode_table_matches_torch_and_closed_forms():
    t = oracle.e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(t, ref, equal_nan=True)
    # closed forms from the format: largest finite, one, smallest normal and subnormal, NaN codes
    assert t[0x7E] == 448.0 and t[0x38] == 1.0 and t[0x08] == 2.0 ** -6 and t[0x01] == 2.0 ** -9
    assert t[0xFE] == -448.0 and t[0x80] == 0.0 and np.signbit(t[0x80])
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.all(np.diff(t[:0x7F]) > 0)  # codes 0..126 ascend


def test_encode_all_bf16_values_match_torch():
    """Every bf16 value in [-448, 448] (the quantizer's inputs when a row's absmax is 448)."""
    bits = np.arange(0, 1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    assert v.size > 30000
    assert np.array_equal(encode(v), torch_encode(v))


def test_encode_ties_and_neighbours_match_torch():
    """Midpoints between adjacent values (ties to even) and the float32 values either side of them."""
    t = oracle.e4m3_table()[:0x7F].astype(np.float64)
    mids = (t[:-1] + t[1:]) / 2
    mids32 = mids.astype(np.float32)
    assert np.array_equal(mids32.astype(np.float64), mids)  # the midpoints are float32-exact
    below = np.nextafter(mids32, np.float32(0))
    above = np.nextafter(mids32, np.float32(np.inf))
    v = np.concatenate([mids32, below, above, -mids32, -below, -above])
    got, ref = encode(v), torch_encode(v)
    assert np.array_equal(got, ref)
    # the tie rule itself: 1 + 1/16 lies between 1 (mantissa 0) and 1.125 (mantissa 1) -> 1
    assert oracle.e4m3_encode(1.0625) == 0x38 and oracle.e4m3_encode(1.1875) == 0x3A


def test_encode_random_and_saturation():
    rng = np.random.default_rng(5)
    v = (rng.choice([-1, 1], 20000) * np.exp2(rng.uniform(-14, np.log2(448), 20000))).astype(np.float32)
    assert np.array_equal(encode(v), torch_encode(v))
    # beyond 448 the quantizer saturates (torch would give NaN past 464)
    assert [oracle.e4m3_encode(x) for x in (448.0, 460.0, 464.0, 1e6, np.inf)] == [0x7E] * 5
    assert oracle.e4m3_encode(-1e6) == 0xFE
    # subnormal ties: 0.5 and 1.5 steps of 2^-9 go to the even neighbours 0 and 2
    assert oracle.e4m3_encode(2.0 ** -10) == 0x00 and oracle.e4m3_encode(3 * 2.0 ** -10) == 0x02


@pytest.mark.parametrize("shape", [(5, 64), (33, 1024)])
def test_quantize_rows_scale_and_error_bound(shape):
    rng = np.random.default_rng(shape[1])
    w = (rng.standard_normal(shape) * np.exp2(rng.uniform(-8, 4, (shape[0], 1)))).astype(np.float32)
    w[0] = 0.0  # a zero row
    w[1, 3] = -50.0  # a row dominated by one value
    q, s = oracle.quantize_e4m3(w)
    amax = np.abs(w).max(1)
    np.testing.assert_array_equal(s, np.where(amax > 0, amax / np.float32(448), 1).astype(np.float32))
    assert np.all(q[0] == 0) and q[1, 3] == 0xFE
    deq = oracle.dequantize_e4m3(q, s)
    # half an ulp of a 3-bit mantissa (2^-4 relative) for normals, half a subnormal step (2^-10 scale) below
    bound = np.maximum(np.abs(w) * 2.0 ** -4, s[:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(np.abs(deq - w) <= bound)
    # the row maxima are exact
    np.testing.assert_allclose(np.abs(deq).max(1)[1:], amax[1:], rtol=1e-6)


def test_known_answer_unit_scale():
    """A row whose absmax is 448 has scale 1 and keeps E4M3-representable values exactly."""
    t = oracle.e4m3_table()
    w = np.array([[448.0, -1.0, 0.5, 2.0 ** -9, -3.5, 0.0, 240.0, -0.013671875]], np.float32)
    q, s = oracle.quantize_e4m3(w)
    assert s[0] == 1.0
    np.testing.assert_array_equal(t[q[0]], w[0])
    assert list(q[0]) == [0x7E, 0xB8, 0x30, 0x01, 0xC6, 0x00, 0x77, 0x87]
