"""Pin the CPU oracle to the golden vectors written from the Hugging Face torch path
(tests/golden/make_golden.py).  The oracle accumulates in fp64 and the vectors are fp32 torch, so the
bar is fp32 rounding noise (rel-L2 <= 2e-6)."""
import os

import numpy as np
import pytest

import oracle

G = os.path.join(os.path.dirname(__file__), "golden")
TOL = 2e-6


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def load(name):
    return dict(np.load(os.path.join(G, name)))


TINY = oracle.dims(256, 2, 4, 32, 32)


@pytest.mark.parametrize("B, T", [(1, 1), (1, 40), (4, 9), (2, 70)])
def test_layer_matches_hf(B, T):
    """The reference's (B, T) grid (9B/test_gdn_layer.py:42-49) plus a chunk-64 boundary crossing."""
    w = load("tiny_weights.npz")
    f = load(f"tiny_layer_B{B}_T{T}.npz")
    rec = np.zeros((B, 4, 32, 32), np.float32)
    conv = np.zeros((B, 256, 3), np.float32)
    out = oracle.layer_forward(TINY, w, f["x"], rec, conv)
    assert rel(out, f["out"]) < TOL
    assert rel(out, f["out_nocache"]) < TOL
    assert rel(rec, f["rec_state"]) < TOL
    assert rel(conv, f["conv_state"]) < TOL


def test_layer_prefill_then_decode_matches_hf():
    """Prefill 20 tokens then 5 single-token calls, state carried (9B/test_gdn_layer.py:52-63)."""
    f = load("tiny_continue.npz")
    rec = np.zeros((1, 4, 32, 32), np.float32)
    conv = np.zeros((1, 256, 3), np.float32)
    outs = [oracle.layer_forward(TINY, f, f["x"][:, :20], rec, conv)]
    outs += [oracle.layer_forward(TINY, f, f["x"][:, t:t + 1], rec, conv) for t in range(20, 25)]
    out = np.concatenate(outs, 1)
    assert rel(out, f["out"]) < TOL
    assert rel(out, f["out_full"]) < TOL
    assert rel(rec, f["rec_state"]) < TOL
    assert rel(conv, f["conv_state"]) < TOL


@pytest.mark.parametrize("name", ["rec_gqa", "rec_real_dims", "rec_slow_decay", "rec_chunk_edge"])
def test_recurrence_matches_hf(name):
    """Sequential and chunk-64 forms against HF's torch_recurrent / torch_chunk rules
    (9B/reference.py:11-35 restates the former; 9B/test_gated_delta_l1.py:48-78 cases)."""
    f = load(name + ".npz")
    init = f.get("init")
    o, s = oracle.recurrent_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], init)
    assert rel(o, f["o"]) < TOL and rel(s, f["state"]) < TOL
    oc, sc = oracle.chunk_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], init)
    assert rel(oc, f["o_chunk"]) < TOL and rel(sc, f["state_chunk"]) < TOL


def test_conv_matches_hf():
    """causal_conv1d_fn (full sequence) and causal_conv1d_update (cached steps), HF:199-239."""
    f = load("conv.npz")
    x = f["x"].transpose(0, 2, 1)  # [1, T, C]
    out, _ = oracle.conv1d_silu(x, f["w"], np.zeros((1, 16, 3), np.float32))
    assert rel(out.transpose(0, 2, 1), f["out_full"]) < TOL
    hist = np.ascontiguousarray(x[:, :3].transpose(0, 2, 1))
    outs, hist = oracle.conv1d_silu(x[:, 3:], f["w"], hist)
    assert rel(outs.transpose(0, 2, 1), f["out_steps"]) < TOL
    assert np.array_equal(hist, f["state_after"])  # history is a copy of inputs: bit-exact


def test_gated_rmsnorm_matches_hf():
    f = load("rmsnorm_gated.npz")
    assert rel(oracle.gated_rmsnorm(f["o"], f["z"], f["w"]), f["y"]) < TOL


def test_planted_tap_reversal_is_caught():
    """A plausible mistake (conv taps applied in the wrong order) must fail the golden check."""
    f = load("conv.npz")
    x = f["x"].transpose(0, 2, 1)
    out, _ = oracle.conv1d_silu(x, f["w"][:, ::-1], np.zeros((1, 16, 3), np.float32))
    assert rel(out.transpose(0, 2, 1), f["out_full"]) > 1e-2
