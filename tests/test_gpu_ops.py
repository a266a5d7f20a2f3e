"""GPU parity of the projection kernels and the recurrence-only op, through the C ABI.

Projections: against an fp64 CPU matmul of the same bf16 operands (fp32 output: accumulation noise
only; bf16 output: one rounding).  Recurrence: the reference's own cases
(9B/test_gated_delta_l1.py:48-92) against the CPU oracle, plus the HF golden vectors; the bar is the
fp32-state tolerance, rel-L2 <= 1e-3, for both the output and the final state.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from linear_attention_op_amd import GatedDeltaRuleHIP, GdnValueError, linear

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

G = os.path.join(os.path.dirname(__file__), "golden")
STATE_TOL = 1e-3


def rel(a, b):
    a = torch.as_tensor(np.asarray(a.cpu() if torch.is_tensor(a) else a), dtype=torch.float64)
    b = torch.as_tensor(np.asarray(b.cpu() if torch.is_tensor(b) else b), dtype=torch.float64)
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("M, N, K", [
    (1, 392, 256), (3, 4096, 4096), (16, 12352, 4096), (17, 1024, 2048), (40, 8224, 1024), (64, 12352, 4096),
    (64, 4096, 4096), (65, 392, 256), (200, 4096, 1024), (512, 12352, 4096), (300, 1000, 128),
    (2048, 8224, 1024), (4096, 4096, 512), (1030, 16400, 256),
])
def test_linear(M, N, K):
    print(f"linear M={M} N={N} K={K}", flush=True)
    gen = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=gen).bfloat16()
    w = (torch.randn(N, K, generator=gen) * 0.02).bfloat16()
    want = x.double() @ w.double().T
    y32 = linear(x.cuda(), w.cuda(), torch.float32)
    y16 = linear(x.cuda(), w.cuda(), torch.bfloat16)
    torch.cuda.synchronize()
    assert rel(y32, want) < 1e-5
    assert rel(y16.float(), want) < 5e-3


def make_rec_inputs(B, T, Hk, Hv, dk, dv, seed=0, g_shift=2.0):
    """The reference's draw order (9B/test_gated_delta_l1.py:17-24)."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hk, dk, generator=gen)
    k = torch.randn(B, T, Hk, dk, generator=gen)
    v = torch.randn(B, T, Hv, dv, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, Hv, generator=gen) + g_shift)
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=gen))
    return q, k, v, g, beta


@pytest.mark.parametrize("B, Hk, Hv, T", [(1, 16, 32, 1), (1, 16, 32, 45), (1, 8, 16, 7), (4, 16, 32, 3)])
def test_recurrence_matches_oracle(B, Hk, Hv, T):
    print(f"recurrence B={B} Hk={Hk} Hv={Hv} T={T}", flush=True)
    dk = dv = 128
    q, k, v, g, beta = make_rec_inputs(B, T, Hk, Hv, dk, dv)
    init = torch.randn(B, Hv, dk, dv) * 0.1
    want_o, want_s = oracle.recurrent_gated_delta_rule(q.numpy(), k.numpy(), v.numpy(), g.numpy(), beta.numpy(),
                                                       init.numpy())
    op = GatedDeltaRuleHIP(B * Hv, dk, dv, initial_state=init.reshape(B * Hv, dk, dv).cuda())
    got_o = op(q, k, v, g, beta)
    torch.cuda.synchronize()
    assert rel(got_o, want_o) < STATE_TOL
    assert rel(op.get_state(), want_s.reshape(B * Hv, dk, dv)) < STATE_TOL


def test_long_sequence_slow_decay():
    """T = 1024 with decay ~0.99 (9B/test_gated_delta_l1.py:69-78)."""
    B, Hk, Hv, dk, dv, T = 1, 16, 32, 128, 128, 1024
    q, k, v, _, beta = make_rec_inputs(B, T, Hk, Hv, dk, dv, seed=3)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, Hv, generator=torch.Generator().manual_seed(4)) + 5.0)
    want_o, want_s = oracle.recurrent_gated_delta_rule(q.numpy(), k.numpy(), v.numpy(), g.numpy(), beta.numpy())
    op = GatedDeltaRuleHIP(B * Hv, dk, dv)
    got_o = op(q, k, v, g, beta)
    torch.cuda.synchronize()
    assert rel(got_o, want_o) < STATE_TOL
    assert rel(op.get_state(), want_s.reshape(B * Hv, dk, dv)) < STATE_TOL


def test_decode_loop_keeps_state_resident():
    """64 single-token calls: the state buffer never moves (9B/test_gated_delta_l1.py:81-92)."""
    B, Hk, Hv, dk, dv, steps = 1, 16, 32, 128, 128, 64
    q, k, v, g, beta = make_rec_inputs(B, steps, Hk, Hv, dk, dv, seed=1)
    want_o, want_s = oracle.recurrent_gated_delta_rule(q.numpy(), k.numpy(), v.numpy(), g.numpy(), beta.numpy())
    op = GatedDeltaRuleHIP(B * Hv, dk, dv)
    addr = op.state.data_ptr()
    outs = [op(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1], beta[:, t:t + 1]) for t in range(steps)]
    assert op.state.data_ptr() == addr
    torch.cuda.synchronize()
    assert rel(torch.cat(outs, 1), want_o) < STATE_TOL
    assert rel(op.get_state(), want_s.reshape(B * Hv, dk, dv)) < STATE_TOL


@pytest.mark.parametrize("name", ["rec_gqa", "rec_real_dims", "rec_slow_decay"])
def test_recurrence_matches_hf_golden(name):
    f = dict(np.load(os.path.join(G, name + ".npz")))
    B, T, Hk, dk = f["q"].shape
    Hv, dv = f["v"].shape[2:]
    init = torch.from_numpy(f["init"]).reshape(B * Hv, dk, dv).cuda() if "init" in f else None
    op = GatedDeltaRuleHIP(B * Hv, dk, dv, initial_state=init)
    o = op(*[torch.from_numpy(f[n]) for n in ("q", "k", "v", "g", "beta")])
    torch.cuda.synchronize()
    assert rel(o, f["o"]) < STATE_TOL
    assert rel(op.get_state(), f["state"].reshape(B * Hv, dk, dv)) < STATE_TOL


@pytest.mark.parametrize("B, Hk, Hv, T, l2", [(1, 16, 32, 65, True), (2, 4, 8, 200, True), (3, 2, 2, 130, False)])
def test_chunked_recurrence_matches_oracle(B, Hk, Hv, T, l2):
    """Launches of more than 64 tokens run the chunk-64 form: ragged tail chunks (65 = 64 + 1, 200, 130), two
    v-heads per k-head, a nonzero initial state, with the op's l2norm and without it (unit q, k and scale 1,
    as the layer hands them over)."""
    print(f"chunked recurrence B={B} Hk={Hk} Hv={Hv} T={T} l2={l2}", flush=True)
    dk = dv = 128
    q, k, v, g, beta = make_rec_inputs(B, T, Hk, Hv, dk, dv, seed=T)
    scale = None
    if not l2:
        q, k, scale = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True), 1.0
    init = torch.randn(B, Hv, dk, dv, generator=torch.Generator().manual_seed(1)) * 0.1
    want_o, want_s = oracle.recurrent_gated_delta_rule(q.numpy(), k.numpy(), v.numpy(), g.numpy(), beta.numpy(),
                                                       init.numpy(), use_qk_l2norm=l2, scale=scale)
    op = GatedDeltaRuleHIP(B * Hv, dk, dv, initial_state=init.reshape(B * Hv, dk, dv).cuda())
    got_o = op(q, k, v, g, beta, use_qk_l2norm=l2, scale=scale)
    torch.cuda.synchronize()
    assert op.workspace is not None  # the chunked form ran
    assert rel(got_o, want_o) < STATE_TOL
    assert rel(op.get_state(), want_s.reshape(B * Hv, dk, dv)) < STATE_TOL


def test_chunked_recurrence_mixed_decay():
    """Chunk decays from ~1 to below 2^-8 within one launch and within one head (the chunked form's W S error
    reaches the state scaled by the chunk's decay): eight v-heads with per-token log decays from -0.004 to -0.3
    and per-token noise, so that 64-token sums fall on both sides of -8 ln 2; against the oracle."""
    print("chunked recurrence, mixed chunk decays", flush=True)
    B, Hk, Hv, dk, dv, T = 1, 4, 8, 128, 128, 640
    gen = torch.Generator().manual_seed(61)
    q = torch.randn(B, T, Hk, dk, generator=gen)
    k = torch.randn(B, T, Hk, dk, generator=gen)
    v = torch.randn(B, T, Hv, dv, generator=gen)
    rate = torch.logspace(np.log10(0.004), np.log10(0.3), Hv)
    g = -rate * (0.2 + 1.6 * torch.rand(B, T, Hv, generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=gen))
    G = g[0].reshape(-1, 64, Hv).sum(1)
    lim = -8 * np.log(2.0)
    # fast and slow chunks overall, and both within one head
    assert (G > lim).any() and (G <= lim).any() and ((G > lim).any(0) & (G <= lim).any(0)).any()
    init = torch.randn(B, Hv, dk, dv, generator=gen) * 0.1
    want_o, want_s = oracle.recurrent_gated_delta_rule(q.numpy(), k.numpy(), v.numpy(), g.numpy(), beta.numpy(),
                                                       init.numpy())
    op = GatedDeltaRuleHIP(B * Hv, dk, dv, initial_state=init.reshape(B * Hv, dk, dv).cuda())
    got_o = op(q, k, v, g, beta)
    torch.cuda.synchronize()
    assert op.workspace is not None  # the chunked form ran
    r_o, r_s = rel(got_o, want_o), rel(op.get_state(), want_s.reshape(B * Hv, dk, dv))
    print(f"  output {r_o:.2e} state {r_s:.2e}", flush=True)
    assert r_o < STATE_TOL and r_s < STATE_TOL


def test_chunked_recurrence_matches_token_loop():
    """9B heads, T = 2048 then T = 100 on the same object (the workspace is kept, the state carried): the
    chunked form against the token loop on the same inputs."""
    B, Hk, Hv, dk, dv = 2, 16, 32, 128, 128
    chunked = GatedDeltaRuleHIP(B * Hv, dk, dv)
    loop = GatedDeltaRuleHIP(B * Hv, dk, dv, chunked=False)
    addr = None
    for T, seed in ((2048, 5), (100, 6)):
        print(f"chunked vs token loop T={T}", flush=True)
        q, k, v, g, beta = make_rec_inputs(B, T, Hk, Hv, dk, dv, seed=seed)
        o_c = chunked(q, k, v, g, beta)
        o_l = loop(q, k, v, g, beta)
        torch.cuda.synchronize()
        assert loop.workspace is None
        addr = addr or chunked.workspace.data_ptr()
        assert chunked.workspace.data_ptr() == addr
        assert rel(o_c, o_l) < STATE_TOL
        assert rel(chunked.get_state(), loop.get_state()) < STATE_TOL


def test_unsupported_head_dims_raise():
    f = dict(np.load(os.path.join(G, "rec_chunk_edge.npz")))  # dk = 16, dv = 24
    B, T, Hk, dk = f["q"].shape
    Hv, dv = f["v"].shape[2:]
    op = GatedDeltaRuleHIP(B * Hv, dk, dv)
    with pytest.raises(GdnValueError):
        op(*[torch.from_numpy(f[n]) for n in ("q", "k", "v", "g", "beta")])


@pytest.mark.parametrize("M", [64, 2048])
def test_in_proj_fragment_weights_against_fp64(M):
    """The layer's in_proj (weights in MFMA-fragment layout; GEMV at M = 64, 256x256-tile GEMM at
    M = 2048) against an fp64 product of the same bf16 operands."""
    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
    from linear_attention_op_amd import synthetic as syn
    d = syn.SHAPES["9b"]
    w, gen = syn.make_weights(d, seed=5)
    layer = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=M)
    x = torch.randn(M, d["hidden"], generator=gen).bfloat16()
    P = layer.in_proj(x.cuda())
    wcat = torch.cat([w["w_qkv"], w["w_z"], w["w_a"], w["w_b"]]).cuda().double()
    want = x.cuda().double() @ wcat.T
    torch.cuda.synchronize()
    assert rel(P, want) < 1e-5
    y = torch.randn(M, d["num_v_heads"] * 128, generator=gen).bfloat16()
    out = layer.out_proj(y.cuda())
    want = y.cuda().double() @ w["w_out"].cuda().double().T
    torch.cuda.synchronize()
    assert rel(out.float(), want) < 5e-3
