"""GPU parity of the MXFP4 weight path (the counterpart of the reference's bfloat4_b), through the C ABI.

Truth: the oracle's MXFP4 quantizer (pinned against the OCP rounding thresholds and closed forms in
test_oracle_fp4.py) and the oracle layer run on the dequantized weights.  Bars: the quantizer's codes and
scale codes bit-exact; projections of one-hot rows on MXFP4-representable weights exact (this pins the W_F4
layout, the scale words and the code -> bf16 widening of every kernel: GEMV, both GEMMs, the decode
in_proj); the layer output rel-L2 <= 1e-2 and the recurrent state <= 1e-3 against the oracle on the same
dequantized weights.
"""
import numpy as np
import pytest
import torch

import oracle
from linear_attention_op_amd import Qwen35GatedDeltaNetHIP, Qwen35GDNStackHIP, quantize_mxfp4
from linear_attention_op_amd import synthetic as syn

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

OUT_TOL = 1e-2
STATE_TOL = 1e-3


def rel(a, b):
    a = np.asarray(a.float().cpu() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b.float().cpu() if torch.is_tensor(b) else b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def odims(d):
    return oracle.dims(d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"])


def packed(q):
    """oracle codes [N, K] (one per byte) -> [N, K / 2], column 2i in the low nibble"""
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def dequantized(w):
    """numpy weights with in_proj_qkv, in_proj_z and out_proj replaced by what the MXFP4 layer multiplies by."""
    wn = syn.to_numpy(w)
    for k in ("w_qkv", "w_z", "w_out"):
        wn[k] = oracle.dequantize_mxfp4(*oracle.quantize_mxfp4(wn[k]))
    return wn


# ---- the quantizer ---------------------------------------------------------------------------------
@pytest.mark.parametrize("N, K", [(64, 4096), (37, 1024), (5, 96)])
def test_quantizer_bit_exact(N, K):
    print(f"quantize N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(N * K)
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    w[0] = 0                   # zero blocks: scale code 0, zero codes
    w[1, :] = 1e-5             # one large value per block: the rest round to zero
    w[1, 7] = -1.0
    w[2] *= 1e4                # large magnitudes
    w[3, :32] = 2.0 ** -130    # a block below the smallest scale (exponent clamped to -127)
    q, s = quantize_mxfp4(w.cuda())
    wq, ws = oracle.quantize_mxfp4(w.float().numpy())
    assert np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(q.cpu().numpy(), packed(wq))


def test_quantizer_every_bf16_value():
    """Blocks led by 6 (scale code 127) holding every bf16 value in [-6, 6]: codes equal the oracle's."""
    bits = np.arange(0, 1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 6)]
    nb = -(-v.size // 31)
    blocks = np.zeros((nb, 32), np.float32)
    blocks[:, 0] = 6.0
    blocks[:, 1:].flat[:v.size] = v
    K = 1024
    rows = -(-nb // (K // 32))
    m = np.zeros((rows * (K // 32), 32), np.float32)
    m[:, 0] = 6.0
    m[:nb] = blocks
    m = m.reshape(rows, K)
    q, s = quantize_mxfp4(torch.from_numpy(m).bfloat16().cuda())
    wq, ws = oracle.quantize_mxfp4(m)
    assert np.all(ws == 127) and np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(q.cpu().numpy(), packed(wq))


# ---- layout and widening: one-hot rows read the weights back exactly ---------------------------------
def representable_weights(d, seed):
    """Weights whose projection rows are MXFP4 values: per 32-column block a grid value times 2^e, the block's
    first element +-6 * 2^e or +-4 * 2^e so that the quantizer picks exactly that scale."""
    g = torch.Generator().manual_seed(seed)
    grid = torch.from_numpy(oracle.e2m1_table())

    def rows(n, k):
        codes = torch.randint(0, 16, (n, k), generator=g)
        m = grid[codes].reshape(n, k // 32, 32)
        lead = torch.where(torch.rand(n, k // 32, generator=g) < 0.5, 6.0, 4.0)
        m[:, :, 0] = lead * torch.where(torch.rand(n, k // 32, generator=g) < 0.5, 1.0, -1.0)
        e = torch.randint(-9, 1, (n, k // 32, 1), generator=g).float()
        return (m * torch.exp2(e)).reshape(n, k)

    w, _ = syn.make_weights(d, seed=seed)
    H, Vd = d["hidden"], d["num_v_heads"] * d["head_v_dim"]
    w["w_qkv"], w["w_z"], w["w_out"] = rows(syn.conv_dim(d), H), rows(Vd, H), rows(H, Vd)
    return w


@pytest.mark.parametrize("M", [5, 64, 1024, 2048])
def test_in_proj_one_hot_rows_exact(M):
    """M <= 64: GEMV; 1024: 128 x 128 GEMM; 2048: 256 x 256 GEMM."""
    print(f"mxfp4 in_proj one-hot M={M}", flush=True)
    d = syn.SHAPES["0.8b"]
    w = representable_weights(d, seed=3)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=64, weight_dtype="mxfp4")
    assert layer.weight_dtype == "mxfp4"
    H = d["hidden"]
    cols = (torch.arange(M) * 37) % H
    x = torch.zeros(M, H)
    x[torch.arange(M), cols] = 1.0
    P = layer.in_proj(x.cuda()).cpu()
    wcat = torch.cat([w["w_qkv"], w["w_z"], w["w_a"].bfloat16().float(), w["w_b"].bfloat16().float()])
    assert torch.equal(P, wcat[:, cols].T.contiguous())


@pytest.mark.parametrize("M", [3, 64, 2048, 16384])
def test_out_proj_one_hot_rows_exact(M):
    """M <= 64: GEMV; 2048: 128 x 128 GEMM; 16384: 256 x 256 GEMM (bf16 output)."""
    print(f"mxfp4 out_proj one-hot M={M}", flush=True)
    d = syn.SHAPES["0.8b"]
    w = representable_weights(d, seed=4)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=64, weight_dtype="mxfp4",
                                  out_dtype=torch.bfloat16)
    Vd = d["num_v_heads"] * d["head_v_dim"]
    cols = (torch.arange(M) * 101) % Vd
    y = torch.zeros(M, Vd)
    y[torch.arange(M), cols] = 1.0
    out = layer.out_proj(y.cuda()).cpu()
    assert torch.equal(out.float(), w["w_out"][:, cols].T.contiguous().bfloat16().float())


def test_decode_in_proj_one_hot_rows_exact():
    """The decode in_proj (MXFP4 rows + split-K bf16 a|b rows) through a whole decode step: with a zero conv
    history and one-hot inputs, the layer's conv history after the step is the q|k|v projection."""
    d = syn.SHAPES["0.8b"]
    w = representable_weights(d, seed=5)
    B = 48
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, weight_dtype="mxfp4")
    H = d["hidden"]
    cols = (torch.arange(B) * 53 + 11) % H
    x = torch.zeros(B, 1, H)
    x[torch.arange(B), 0, cols] = 1.0
    layer(x.cuda())
    conv = layer.get_conv_state().cpu()
    assert torch.equal(conv[:, :, 2], w["w_qkv"][:, cols].T.contiguous())
    assert torch.all(conv[:, :, :2] == 0)


# ---- the layer against the oracle on dequantized weights --------------------------------------------
def run(layer, d, wn, x, s0, steps):
    """`steps` launches of x split evenly along T; -> worst out and final state errors against the oracle."""
    B, T = x.shape[:2]
    rec_o = s0.numpy().copy()
    conv_o = np.zeros((B, syn.conv_dim(d), 3), np.float32)
    layer.set_state(rec=s0.cuda())
    worst = 0.0
    xg = x.cuda()
    for c in torch.arange(T).chunk(steps):
        t0, t1 = int(c[0]), int(c[-1]) + 1
        out = layer(xg[:, t0:t1])
        want = oracle.layer_forward(odims(d), wn, x[:, t0:t1].numpy(), rec_o, conv_o)
        worst = max(worst, rel(out, want))
    return worst, rel(layer.get_recurrent_state(), rec_o)


@pytest.mark.parametrize("shape, B, T, steps", [("0.8b", 4, 3, 3), ("9b", 64, 2, 2), ("9b", 1, 256, 1),
                                                ("0.8b", 1, 2048, 1), ("0.8b", 2, 40, 1)])
def test_layer_matches_oracle_on_dequantized_weights(shape, B, T, steps):
    print(f"mxfp4 layer {shape} B={B} T={T}", flush=True)
    d = syn.SHAPES[shape]
    w, gen = syn.make_weights(d, seed=21)
    x, s0 = syn.make_inputs(d, B, T, gen, state_std=0.01)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, weight_dtype="mxfp4")
    out_err, state_err = run(layer, d, dequantized(w), x, s0, steps)
    print(f"  out {out_err:.2e} state {state_err:.2e}", flush=True)
    assert out_err < OUT_TOL
    assert state_err < STATE_TOL


def test_mxfp4_error_against_bf16_weights():
    """The quantization error itself: the MXFP4 layer's decode output against the oracle on the unquantized
    weights, 9B shape, B = 8.  E2M1 keeps one mantissa bit under a power-of-two scale per 32 weights (~11 %
    rms error per weight on these N(0, 0.02) weights); recorded, with a bound that only catches a broken path."""
    d = syn.SHAPES["9b"]
    w, gen = syn.make_weights(d, seed=22)
    x, s0 = syn.make_inputs(d, 8, 1, gen, state_std=0.01)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=8, weight_dtype="mxfp4")
    err, _ = run(layer, d, syn.to_numpy(w), x, s0, 1)
    print(f"mxfp4 vs bf16 weights: out rel-L2 {err:.3e}", flush=True)
    assert err < 0.35


def test_mxfp4_stack_equals_chained_layers():
    d = syn.SHAPES["0.8b"]
    ws = [syn.make_weights(d, seed=30 + i)[0] for i in range(3)]
    B = 4
    x, _ = syn.make_inputs(d, B, 2, torch.Generator().manual_seed(9))
    st = Qwen35GDNStackHIP(ws, dims=d, batch=B, weight_dtype="mxfp4")
    layers = [Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, max_tokens=64, weight_dtype="mxfp4") for w in ws]
    xg = x.cuda()
    for t in range(2):
        got = st(xg[:, t:t + 1])
        h = xg[:, t:t + 1]
        for lay in layers:
            h = lay(h)
        assert torch.equal(got, h)
