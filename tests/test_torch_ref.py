"""The fp32 torch-CPU restatement timed as the CPU baseline (oracle/torch_ref.py) computes the layer: against
the HF golden vectors (its chunk-64 prefill and its per-token decode) and against the fp64 oracle at the
0.8B shape with GQA-free and GQA geometries.  fp32 against fp64 / fp32 torch: rel-L2 <= 1e-4."""
import os

import numpy as np
import pytest
import torch

import oracle
from linear_attention_op_amd import synthetic as syn
from oracle.torch_ref import GDNLayerTorchCPU

G = os.path.join(os.path.dirname(__file__), "golden")
TOL = 1e-4


def rel(a, b):
    a = np.asarray(a.detach().numpy() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().numpy() if torch.is_tensor(b) else b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def load(name):
    return dict(np.load(os.path.join(G, name)))


@pytest.mark.parametrize("B, T", [(1, 40), (2, 70)])
def test_prefill_and_decode_match_hf(B, T):
    """Prefill of each sequence (chunk-64 form, T = 70 crosses a chunk), and the same tokens one decode step
    at a time, against HF's layer output and final states."""
    w = load("tiny_weights.npz")
    f = load(f"tiny_layer_B{B}_T{T}.npz")
    lay = GDNLayerTorchCPU(w, syn.SHAPES["tiny"])
    x = torch.from_numpy(f["x"])
    for b in range(B):
        rec, conv = torch.zeros(4, 32, 32), torch.zeros(256, 3)
        out = lay.prefill(x[b], rec, conv)
        assert rel(out, f["out"][b]) < TOL
        assert rel(rec, f["rec_state"][b]) < TOL
        assert rel(conv, f["conv_state"][b]) < TOL
    rec, conv = torch.zeros(B, 4, 32, 32), torch.zeros(B, 256, 3)
    out = torch.stack([lay.decode(x[:, t], rec, conv) for t in range(T)], 1)
    assert rel(out, f["out"]) < TOL
    assert rel(rec, f["rec_state"]) < TOL


@pytest.mark.parametrize("shape", ["0.8b", "tiny_gqa"])
def test_against_oracle(shape):
    """Decode from a nonzero state (3 steps, B = 3) and a ragged 150-token prefill against the fp64 oracle."""
    d = dict(syn.SHAPES["tiny"], num_v_heads=8) if shape == "tiny_gqa" else syn.SHAPES[shape]
    w, gen = syn.make_weights(d, seed=7)
    wn = syn.to_numpy(w)
    dm = oracle.dims(d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"])
    lay = GDNLayerTorchCPU(w, d)
    B, C = 3, syn.conv_dim(d)
    x, s0 = syn.make_inputs(d, B, 3, gen, state_std=0.01)
    rec, conv = s0.clone(), torch.zeros(B, C, 3)
    rec_o, conv_o = s0.numpy().copy(), np.zeros((B, C, 3), np.float32)
    for t in range(3):
        got = lay.decode(x[:, t], rec, conv)
        want = oracle.layer_forward(dm, wn, x[:, t:t + 1].numpy(), rec_o, conv_o)[:, 0]
        assert rel(got, want) < TOL, f"step {t}"
    assert rel(rec, rec_o) < TOL and rel(conv, conv_o) < TOL
    xp, _ = syn.make_inputs(d, 1, 150, gen)
    rec, conv = s0[0].clone(), torch.zeros(C, 3)
    rec_o, conv_o = s0[:1].numpy().copy(), np.zeros((1, C, 3), np.float32)
    got = lay.prefill(xp[0], rec, conv)
    want = oracle.layer_forward(dm, wn, xp.numpy(), rec_o, conv_o)[0]
    assert rel(got, want) < TOL
    assert rel(rec, rec_o[0]) < TOL and rel(conv, conv_o[0]) < TOL
