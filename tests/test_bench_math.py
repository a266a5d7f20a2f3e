"""The roofline numerators of bench.py: algorithmic bytes of a decode step and of the mixer launch, FLOPs of a
prefill token.  The bf16 figures are pinned to the values derived by hand from the layer's shapes (9B: W =
134,807,552 B, s = 4,341,760 B per sequence; 0.8B: 21,086,208 and 2,199,552; 140,596,565 FLOP per 9B prefill
token); the low-precision weight bytes to a count of every stored array written out separately."""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402
from linear_attention_op_amd import synthetic as syn  # noqa: E402

D9, D08 = syn.SHAPES["9b"], syn.SHAPES["0.8b"]
S9 = 4_341_760  # per-sequence bytes at 9B: fp32 state read + write, conv history, x and out


def test_decode_bytes_bf16():
    assert bench.decode_bytes(D9, 64) == (134_807_552, S9)
    assert bench.decode_bytes(D08, 1) == (21_086_208, 2_199_552)
    W, s = bench.decode_bytes(D9, 64)
    assert W + 64 * s == 412_680_192


def test_decode_bytes_low_precision():
    H, nk, nv, dk, dv = D9["hidden"], D9["num_k_heads"], D9["num_v_heads"], D9["head_k_dim"], D9["head_v_dim"]
    conv_dim, Vd = 2 * nk * dk + nv * dv, nv * dv
    in_rows, out_rows = conv_dim + Vd, H              # in_proj q|k|v|z rows, out_proj rows
    codes = in_rows * H + out_rows * Vd               # weights held as codes
    ab, taps = 2 * nv * H * 2, conv_dim * 4 * 2       # a|b rows and conv taps, bf16 in every format
    expect = {
        "fp8": codes + 4 * (in_rows + out_rows) + ab + taps,        # 1-byte codes, an fp32 scale per row
        "mxfp4": codes // 2 + codes // 32 + ab + taps,              # 4-bit codes, a 1-byte scale per 32
        "mxint8": codes + codes // 32 + ab + taps,                  # 1-byte codes, a 1-byte scale per 32
    }
    for fmt, want in expect.items():
        assert bench.decode_bytes(D9, 64, fmt) == (want, S9), fmt
    # the per-step figures the bench lines of these formats carry
    assert bench.decode_bytes(D9, 64, "fp8")[0] + 64 * S9 == 345_636_864
    assert bench.decode_bytes(D9, 64, "mxfp4")[0] + 64 * S9 == 314_114_048


def test_mixer_bytes_and_prefill_flops():
    assert 64 * bench.mixer_bytes_per_seq(D9) == 280_510_464
    assert round(bench.prefill_flops_per_token(D9)) == 140_596_565
    assert abs(bench.prefill_flops_per_token(D9) * 16384 - 2.3035e12) < 1e8
