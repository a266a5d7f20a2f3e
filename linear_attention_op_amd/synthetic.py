"""Deterministic synthetic weights and inputs for the GDN layer shapes (no checkpoints, no network).

Draw order, all from one torch CPU generator seeded with `seed` (the reference's convention of one
seeded generator, wormhole_n150/qwen3.5_9B/test_gated_delta_l1.py:17-24):
    w_qkv [conv_dim, H], w_z [Vd, H], w_a [nv, H], w_b [nv, H], conv_w [conv_dim, 4], w_out [H, Vd]
        ~ N(0, 0.02), rounded to bf16 (values kept as float32 here);
    norm_w [dv] ~ U(0.5, 1.5), dt_bias [nv] ~ U(-1, 1)      (9B/test_gdn_layer.py:23-24)
    A_log [nv] = log(U(0, 16))                               (HF Qwen3_5GatedDeltaNet init)
then, from the same generator, layer inputs: x [B, T, H] ~ N(0, 1) rounded to bf16 and, when asked,
the initial recurrent state S0 [B, nv, dk, dv] ~ N(0, state_std).
"""

import torch

SHAPES = {
    # Qwen3.5-0.8B-like GDN layer
    "0.8b": dict(hidden=1024, num_k_heads=16, num_v_heads=16, head_k_dim=128, head_v_dim=128, conv_kernel=4,
                 rms_norm_eps=1e-6),
    # Qwen3.5-9B-like GDN layer
    "9b": dict(hidden=4096, num_k_heads=16, num_v_heads=32, head_k_dim=128, head_v_dim=128, conv_kernel=4,
               rms_norm_eps=1e-6),
    # tiny geometry of the golden vectors
    "tiny": dict(hidden=256, num_k_heads=2, num_v_heads=4, head_k_dim=32, head_v_dim=32, conv_kernel=4,
                 rms_norm_eps=1e-6),
}


def conv_dim(d):
    return 2 * d["num_k_heads"] * d["head_k_dim"] + d["num_v_heads"] * d["head_v_dim"]


def make_weights(dims, seed, gen=None):
    """Weights dict (float32 CPU tensors, projection weights bf16-valued) and the generator, for reuse."""
    g = gen or torch.Generator().manual_seed(seed)
    H, nv, dv = dims["hidden"], dims["num_v_heads"], dims["head_v_dim"]
    C, Vd = conv_dim(dims), nv * dv

    def n(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).bfloat16().float()

    w = {"w_qkv": n(C, H), "w_z": n(Vd, H), "w_a": n(nv, H), "w_b": n(nv, H), "conv_w": n(C, 4), "w_out": n(H, Vd)}
    w["norm_w"] = torch.rand(dv, generator=g) + 0.5
    w["dt_bias"] = torch.rand(nv, generator=g) * 2.0 - 1.0
    w["A_log"] = torch.log(torch.rand(nv, generator=g) * 16.0).clamp_min(-20.0)
    return w, g


def make_inputs(dims, B, T, gen, state_std=None):
    """x [B, T, H] bf16-valued float32 and, if state_std is given, S0 [B, nv, dk, dv] float32."""
    x = torch.randn(B, T, dims["hidden"], generator=gen).bfloat16().float()
    s0 = None
    if state_std is not None:
        s0 = torch.randn(B, dims["num_v_heads"], dims["head_k_dim"], dims["head_v_dim"], generator=gen) * state_std
    return x, s0


def to_numpy(w):
    return {k: v.float().numpy() for k, v in w.items()}


def continuous_batch(dims, n_layers=24, n_prefill=8, prefill_len=2048, n_decode=56, seed=4, device="cuda"):
    """The continuous-batching stack workload: `n_layers` layers and one step of `n_prefill` prompts of
    `prefill_len` tokens followed by `n_decode` single-token streams (sequence i on slot i).

    Drawn on the device from one torch generator seeded with `seed` (a CPU draw of 24 9B-shape layers takes
    minutes): per layer w_qkv, w_z, w_a, w_b, conv_w, w_out ~ N(0, 0.02) rounded to bf16; then, from a CPU
    generator with the same seed, norm_w, dt_bias, A_log of every layer as in make_weights; then the decode
    streams' states S0 [n_decode, nv, dk, dv] ~ N(0, 0.01) for every layer (a GDN state has a fixed size, so
    a long context changes only its values), and the step's input rows x [rows, H] ~ N(0, 1) in bf16.
    Returns (layers: list of weight dicts, cu_seqlens: list, x, s0: list per layer)."""
    dev = torch.device(device)
    gg = torch.Generator(device=dev).manual_seed(seed)
    gc = torch.Generator().manual_seed(seed)
    H, nv, dk, dv = dims["hidden"], dims["num_v_heads"], dims["head_k_dim"], dims["head_v_dim"]
    C, Vd = conv_dim(dims), nv * dv

    def n(*shape):
        return (torch.randn(*shape, generator=gg, device=dev) * 0.02).to(torch.bfloat16)

    layers = []
    for _ in range(n_layers):
        layers.append({"w_qkv": n(C, H), "w_z": n(Vd, H), "w_a": n(nv, H), "w_b": n(nv, H),
                       "conv_w": n(C, 4).float(), "w_out": n(H, Vd)})
    for w in layers:
        w["norm_w"] = torch.rand(dv, generator=gc) + 0.5
        w["dt_bias"] = torch.rand(nv, generator=gc) * 2.0 - 1.0
        w["A_log"] = torch.log(torch.rand(nv, generator=gc) * 16.0).clamp_min(-20.0)
    s0 = [torch.randn(n_decode, nv, dk, dv, generator=gg, device=dev) * 0.01 for _ in range(n_layers)]
    cu = [0]
    for i in range(n_prefill + n_decode):
        cu.append(cu[-1] + (prefill_len if i < n_prefill else 1))
    x = torch.randn(cu[-1], H, generator=gg, device=dev).to(torch.bfloat16)
    return layers, cu, x, s0
