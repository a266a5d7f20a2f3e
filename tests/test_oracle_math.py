"""Closed forms, invariants and integer rules that pin the CPU oracle independently of the golden
vectors.  Each check is chosen so that a plausible mistake (a dropped term, a wrong sign or index, a
transposed operand, tile instead of repeat_interleave) fails it."""
import numpy as np
import pytest

import oracle


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def rng(seed):
    return np.random.default_rng(seed)


# ---- integer rules ---------------------------------------------------------------------------------
def test_khead_mapping_is_repeat_interleave():
    # 9B: nv=32, nk=16 -> h // 2 (gdn_layer.py:51); 0.8B: identity
    assert [oracle.khead_of_vhead(h, 32, 16) for h in range(32)] == [h // 2 for h in range(32)]
    assert [oracle.khead_of_vhead(h, 16, 16) for h in range(16)] == list(range(16))
    assert [oracle.khead_of_vhead(h, 8, 2) for h in range(8)] == [0, 0, 0, 0, 1, 1, 1, 1]


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 9, 128])
def test_conv_shift_and_roll_tables(T):
    """layer_reader.cpp:111-120 (shift) and :189-194 (roll), written out as explicit tables."""
    for t in range(T):
        for s in (1, 2, 3):
            want = t - s if t >= s else -((3 + t - s) + 1)
            assert oracle.conv_src(t, s, T) == want
    for k in range(3):
        want = T + k - 3 if T + k >= 3 else -((T + k) + 1)
        assert oracle.roll_src(T, k) == want
    # T = 1: new history = [old1, old2, x0]; T = 2: [old2, x0, x1]
    if T == 1:
        assert [oracle.roll_src(1, k) for k in range(3)] == [-2, -3, 0]
    if T == 2:
        assert [oracle.roll_src(2, k) for k in range(3)] == [-3, 0, 1]


def test_row_to_bt_sequence_major():
    for T in (1, 3, 7):
        for m in range(4 * T):
            assert oracle.row_to_bt(m, T) == (m // T, m % T)


# ---- projections -------------------------------------------------------------------------------------
def test_linear_against_fp64_matmul():
    r = rng(0)
    x = r.standard_normal((5, 37)).astype(np.float32)
    w = r.standard_normal((11, 37)).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert rel(oracle.linear(x, w), want) < 1e-7
    # transposed operand would give the wrong shape or values
    assert oracle.linear(x, w).shape == (5, 11)


# ---- conv --------------------------------------------------------------------------------------------
def silu(x):
    return x / (1.0 + np.exp(-x))


def test_conv_delta_input_returns_reversed_taps():
    """A unit impulse at t=0 with zero history: pre-activation output at t is w[:, 3 - t]."""
    C, T = 3, 5
    w = rng(1).standard_normal((C, 4)).astype(np.float32)
    x = np.zeros((1, T, C), np.float32)
    x[0, 0, :] = 1.0
    out, _ = oracle.conv1d_silu(x, w, np.zeros((1, C, 3), np.float32))
    for t in range(T):
        want = silu(w[:, 3 - t].astype(np.float64)) if t <= 3 else np.zeros(C)
        assert rel(out[0, t], want) < 1e-7 or np.allclose(out[0, t], want, atol=1e-12)


def test_conv_matches_numpy_convolution():
    r = rng(2)
    C, T = 4, 9
    w = r.standard_normal((C, 4)).astype(np.float32)
    x = r.standard_normal((1, T, C)).astype(np.float32)
    hist = r.standard_normal((1, C, 3)).astype(np.float32)
    out, new_hist = oracle.conv1d_silu(x, w, hist)
    for ch in range(C):
        seq = np.concatenate([hist[0, ch].astype(np.float64), x[0, :, ch].astype(np.float64)])
        full = np.convolve(seq, w[ch, ::-1].astype(np.float64), mode="valid")  # correlation with w
        assert rel(out[0, :, ch], silu(full)) < 1e-7
        assert np.array_equal(new_hist[0, ch], seq[-3:].astype(np.float32))


@pytest.mark.parametrize("split", [1, 2, 3, 5])
def test_conv_launch_split_is_bit_exact(split):
    """Running T tokens as two launches with the history carried equals one launch, bit for bit."""
    r = rng(3)
    C, T = 6, 8
    w = r.standard_normal((C, 4)).astype(np.float32)
    x = r.standard_normal((2, T, C)).astype(np.float32)
    h0 = r.standard_normal((2, C, 3)).astype(np.float32)
    full, hf = oracle.conv1d_silu(x, w, h0)
    a, ha = oracle.conv1d_silu(x[:, :split], w, h0)
    b, hb = oracle.conv1d_silu(x[:, split:], w, ha)
    assert np.array_equal(np.concatenate([a, b], 1), full)
    assert np.array_equal(hb, hf)


# ---- recurrence invariants ---------------------------------------------------------------------------
def rec_inputs(B, T, Hk, Hv, dk, dv, seed):
    r = rng(seed)
    q = r.standard_normal((B, T, Hk, dk)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, dk)).astype(np.float32)
    v = r.standard_normal((B, T, Hv, dv)).astype(np.float32)
    g = np.log(1 / (1 + np.exp(-(r.standard_normal((B, T, Hv)) + 2)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-r.standard_normal((B, T, Hv))))).astype(np.float32)
    return q, k, v, g, beta


def l2n(x):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)


def test_no_decay_no_write_reads_state():
    """g = 0 and beta = 0: S is unchanged and o = S^T q_hat."""
    B, T, Hk, Hv, dk, dv = 1, 3, 1, 2, 8, 6
    q, k, v, _, _ = rec_inputs(B, T, Hk, Hv, dk, dv, 4)
    S0 = rng(5).standard_normal((B, Hv, dk, dv)).astype(np.float32)
    g = np.zeros((B, T, Hv), np.float32)
    beta = np.zeros((B, T, Hv), np.float32)
    o, s = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, S0)
    assert rel(s, S0) < 1e-7
    qh = l2n(q) * dk ** -0.5
    for h in range(Hv):
        want = np.einsum("tk,kv->tv", qh[0, :, 0], S0[0, h].astype(np.float64))
        assert rel(o[0, :, h], want) < 1e-6


def test_full_decay_resets_state():
    """g -> -inf (exp(g) = 0): one token leaves S = k_hat (beta v)^T."""
    B, T, Hk, Hv, dk, dv = 1, 1, 1, 1, 8, 5
    q, k, v, _, beta = rec_inputs(B, T, Hk, Hv, dk, dv, 6)
    S0 = rng(7).standard_normal((B, Hv, dk, dv)).astype(np.float32)
    g = np.full((B, T, Hv), -1e4, np.float32)
    _, s = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, S0)
    want = np.outer(l2n(k)[0, 0, 0], beta[0, 0, 0] * v[0, 0, 0].astype(np.float64))
    assert rel(s[0, 0], want) < 1e-6


def test_unit_beta_stores_value_exactly():
    """beta = 1: the new state maps k_hat to v (delta rule with a unit key; |k_hat|^2 = 1 - O(1e-6))."""
    B, T, Hk, Hv, dk, dv = 1, 1, 1, 1, 16, 7
    q, k, v, g, _ = rec_inputs(B, T, Hk, Hv, dk, dv, 8)
    k *= 10.0  # |k|^2 >> eps, so |k_hat| = 1 to ~1e-9
    S0 = rng(9).standard_normal((B, Hv, dk, dv)).astype(np.float32)
    beta = np.ones((B, T, Hv), np.float32)
    _, s = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, S0)
    kh = l2n(k)[0, 0, 0]
    assert rel(kh @ s[0, 0].astype(np.float64), v[0, 0, 0]) < 1e-5


def test_heads_and_value_columns_are_independent():
    """Changing v of head 1, column 3 changes only (head 1, column 3) of o and S."""
    B, T, Hk, Hv, dk, dv = 1, 4, 1, 2, 8, 6
    q, k, v, g, beta = rec_inputs(B, T, Hk, Hv, dk, dv, 10)
    o1, s1 = oracle.recurrent_gated_delta_rule(q, k, v, g, beta)
    v2 = v.copy()
    v2[:, :, 1, 3] += 1.0
    o2, s2 = oracle.recurrent_gated_delta_rule(q, k, v2, g, beta)
    diff_o = np.abs(o2 - o1).sum(axis=(0, 1))  # [Hv, dv]
    diff_s = np.abs(s2 - s1).sum(axis=(0, 2))  # [Hv, dv]
    mask = np.zeros((Hv, dv), bool)
    mask[1, 3] = True
    assert np.all(diff_o[~mask] == 0) and diff_o[1, 3] > 0
    assert np.all(diff_s[~mask] == 0) and diff_s[1, 3] > 0


def test_gqa_uses_repeat_interleave():
    """With Hk = 2, Hv = 4, v-heads 0,1 read k-head 0 and v-heads 2,3 read k-head 1 (not h % Hk)."""
    B, T, Hk, Hv, dk, dv = 1, 3, 2, 4, 8, 4
    q, k, v, g, beta = rec_inputs(B, T, Hk, Hv, dk, dv, 11)
    o1, _ = oracle.recurrent_gated_delta_rule(q, k, v, g, beta)
    q2 = q.copy()
    q2[:, :, 1] *= -1.0  # flip k-head 1's query
    o2, _ = oracle.recurrent_gated_delta_rule(q2, k, v, g, beta)
    changed = [bool(np.any(o1[:, :, h] != o2[:, :, h])) for h in range(Hv)]
    assert changed == [False, False, True, True]


@pytest.mark.parametrize("T, chunk", [(1, 64), (63, 64), (64, 64), (65, 64), (200, 64), (37, 16)])
def test_chunked_equals_sequential(T, chunk):
    """The chunk (WY/UT) form is an identity of the sequential rule (HF:248-328 vs reference.py:11-35)."""
    B, Hk, Hv, dk, dv = 2, 2, 4, 16, 8
    q, k, v, g, beta = rec_inputs(B, T, Hk, Hv, dk, dv, 12)
    S0 = (rng(13).standard_normal((B, Hv, dk, dv)) * 0.1).astype(np.float32)
    o, s = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, S0)
    oc, sc = oracle.chunk_gated_delta_rule(q, k, v, g, beta, S0, chunk=chunk)
    assert rel(oc, o) < 1e-6 and rel(sc, s) < 1e-6


def test_scale_and_l2norm_flags():
    """use_qk_l2norm=False with pre-normalised inputs equals the default; an explicit scale of dk^-0.5
    equals the default scale."""
    B, T, Hk, Hv, dk, dv = 1, 5, 1, 1, 8, 4
    q, k, v, g, beta = rec_inputs(B, T, Hk, Hv, dk, dv, 14)
    o1, s1 = oracle.recurrent_gated_delta_rule(q, k, v, g, beta)
    o2, s2 = oracle.recurrent_gated_delta_rule(l2n(q), l2n(k), v, g, beta, use_qk_l2norm=False)
    o3, _ = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, scale=dk ** -0.5)
    assert rel(o2, o1) < 1e-6 and rel(s2, s1) < 1e-6 and rel(o3, o1) < 1e-7


# ---- gated RMSNorm ------------------------------------------------------------------------------------
def test_rmsnorm_constant_input():
    """o = c * 1 gives y = w * silu(z) (rstd * c = 1 up to eps)."""
    dv = 16
    r = rng(15)
    w = r.uniform(0.5, 1.5, dv).astype(np.float32)
    z = r.standard_normal((3, dv)).astype(np.float32)
    o = np.full((3, dv), 2.5, np.float32)
    y = oracle.gated_rmsnorm(o, z, w)
    assert rel(y, w * silu(z.astype(np.float64))) < 1e-6


def test_rmsnorm_scale_invariant():
    dv = 16
    r = rng(16)
    w = r.uniform(0.5, 1.5, dv).astype(np.float32)
    z = r.standard_normal((4, dv)).astype(np.float32)
    o = r.standard_normal((4, dv)).astype(np.float32)
    assert rel(oracle.gated_rmsnorm(7.0 * o, z, w), oracle.gated_rmsnorm(o, z, w)) < 1e-6
