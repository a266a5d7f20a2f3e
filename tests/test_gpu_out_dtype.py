"""Output element type of the layer and the stack, through the C ABI.

The reference returns fp32: its layer computes out_proj with dtype=ttnn.float32 (9B/gdn_layer.py:272-276) and
its stack returns fp32 rows (0.8B/gdn_l1.py:300, 336-339).  Both output types store the same fp32 sums of the
out_proj, so on every projection path (row-major and fragment GEMVs, both GEMMs, bf16 and E4M3 weights, split
and variable-length launches, the stack) the bf16 output must equal the fp32 output rounded to nearest even,
bit for bit, with the states unchanged; the fp32 output is checked against the oracle (rel-L2 <= 1e-2, and no
further from it than the bf16 output) and, for the projection alone, against an fp64 product (<= 1e-5).
"""
import numpy as np
import pytest
import torch

import oracle
from linear_attention_op_amd import Qwen35GatedDeltaNetHIP, Qwen35GDNStackHIP
from linear_attention_op_amd import synthetic as syn

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

OUT_TOL = 1e-2


def rel(a, b):
    a = np.asarray(a.float().cpu() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b.float().cpu() if torch.is_tensor(b) else b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def odims(d):
    return oracle.dims(d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"])


def pair(w, d, B, max_tokens, weight_dtype="bf16"):
    """The same layer twice: fp32 output, bf16 output."""
    return [Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, max_tokens=max_tokens, weight_dtype=weight_dtype,
                                   out_dtype=dt) for dt in (torch.float32, torch.bfloat16)]


def check_rounding(out32, out16):
    assert out32.dtype == torch.float32 and out16.dtype == torch.bfloat16
    assert torch.equal(out32.to(torch.bfloat16), out16)


# (shape, B, T, weight dtype, oracle): decode through the row-major GEMV (B <= 16) and the fragment GEMV
# (B = 64), prefill through the 128 x 128 GEMM (M = 300) and the 256 x 256 GEMM (9B, M = 4096)
CASES = [
    ("0.8b", 4, 1, "bf16", True),
    ("0.8b", 1, 300, "bf16", True),
    ("0.8b", 4, 1, "fp8", False),
    ("0.8b", 1, 300, "fp8", False),
    ("9b", 64, 1, "bf16", False),
    ("9b", 1, 4096, "bf16", False),
]


@pytest.mark.parametrize("shape, B, T, wd, use_oracle", CASES)
def test_fp32_output_rounds_to_bf16_output(shape, B, T, wd, use_oracle):
    print(f"out dtype {shape} B={B} T={T} {wd}", flush=True)
    d = syn.SHAPES[shape]
    w, gen = syn.make_weights(d, seed=8)
    x, s0 = syn.make_inputs(d, B, T, gen, state_std=0.01)
    a, b = pair(w, d, B, max(64, B * T), wd)
    for lay in (a, b):
        lay.set_state(rec=s0.cuda())
    xg = x.cuda()
    out32, out16 = a(xg), b(xg)
    torch.cuda.synchronize()
    check_rounding(out32, out16)
    assert torch.equal(a.get_recurrent_state(), b.get_recurrent_state())
    assert torch.equal(a.get_conv_state(), b.get_conv_state())
    if use_oracle:
        rec = s0.numpy().astype(np.float32).copy()
        conv = np.zeros((B, syn.conv_dim(d), 3), np.float32)
        want = oracle.layer_forward(odims(d), syn.to_numpy(w), x.numpy(), rec, conv)
        r32, r16 = rel(out32, want), rel(out16, want)
        print(f"  rel to oracle: fp32 {r32:.3e}, bf16 {r16:.3e}", flush=True)
        assert r32 < OUT_TOL and r32 <= r16


@pytest.mark.parametrize("B", [1, 2])
def test_split_launch_fp32_output(B):
    """T > max_tokens / B: token blocks of 32 rows; B = 2 gathers each block's fp32 rows in the projection
    workspace before scattering them to the sequences."""
    print(f"out dtype split launch B={B}", flush=True)
    d = syn.SHAPES["0.8b"]
    w, gen = syn.make_weights(d, seed=9)
    T = 100
    x, _ = syn.make_inputs(d, B, T, gen)
    a, b = pair(w, d, B, 32 * B)
    xg = x.cuda()
    out32, out16 = a(xg), b(xg)
    torch.cuda.synchronize()
    check_rounding(out32, out16)
    rec = np.zeros((B, d["num_v_heads"], 128, 128), np.float32)
    conv = np.zeros((B, syn.conv_dim(d), 3), np.float32)
    want = oracle.layer_forward(odims(d), syn.to_numpy(w), x.numpy(), rec, conv)
    assert rel(out32, want) < OUT_TOL
    assert rel(a.get_recurrent_state(), rec) < 1e-3


def test_varlen_fp32_output():
    print("out dtype varlen", flush=True)
    d = syn.SHAPES["0.8b"]
    w, gen = syn.make_weights(d, seed=10)
    cu = [0, 1, 5, 70, 71]
    x = torch.randn(cu[-1], d["hidden"], generator=gen).bfloat16().cuda()
    a, b = pair(w, d, 4, 128)
    out32, out16 = a.forward_varlen(x, cu), b.forward_varlen(x, cu)
    torch.cuda.synchronize()
    check_rounding(out32, out16)
    assert torch.equal(a.get_recurrent_state(), b.get_recurrent_state())


@pytest.mark.parametrize("M", [3, 64, 2048, 16384])
def test_out_proj_fp32_against_fp64(M):
    """Per-op out_proj with fp32 output: GEMV (M <= 64), 128 x 128 GEMM, 256 x 256 GEMM, against the fp64
    product of the same bf16 operands (9B/gdn_layer.py:272-276)."""
    print(f"out_proj fp32 M={M}", flush=True)
    d = syn.SHAPES["0.8b"]
    w, gen = syn.make_weights(d, seed=11)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=64)
    y = torch.randn(M, d["num_v_heads"] * 128, generator=gen).bfloat16()
    out = layer.out_proj(y.cuda())
    want = y.cuda().double() @ w["w_out"].cuda().double().T
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    assert rel(out, want) < 1e-5


def test_stack_fp32_output():
    """The stack's last layer writes fp32; calls that end before it, and the activations between layers, are
    bf16; a split launch of two sequences (T > max_tokens / B) gathers its fp32 rows in the workspace."""
    print("out dtype stack", flush=True)
    d = syn.SHAPES["0.8b"]
    gen = torch.Generator().manual_seed(12)
    ws = [syn.make_weights(d, seed=None, gen=gen)[0] for _ in range(3)]
    B = 2
    s32 = Qwen35GDNStackHIP(ws, dims=d, batch=B, max_tokens=64, inter_norm=True, out_dtype=torch.float32)
    s16 = Qwen35GDNStackHIP(ws, dims=d, batch=B, max_tokens=64, inter_norm=True, out_dtype=torch.bfloat16)
    for T in (1, 7, 40):
        x = torch.randn(B, T, d["hidden"], generator=gen).bfloat16().cuda()
        out32, out16 = s32(x), s16(x)
        torch.cuda.synchronize()
        check_rounding(out32, out16)
        for i in range(3):
            assert torch.equal(s32.get_recurrent_state(i), s16.get_recurrent_state(i)), (T, i)
    # layers 0 and 1 only: bf16 activations after layer 1 (widened to the stack's output type)
    x = torch.randn(B, 1, d["hidden"], generator=gen).bfloat16().cuda()
    sub32, sub16 = s32(x, layers=[0, 1]), s16(x, layers=[0, 1])
    torch.cuda.synchronize()
    assert sub32.dtype == torch.float32 and torch.equal(sub32, sub16.float())
