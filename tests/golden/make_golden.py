"""Write the golden vectors that pin the CPU oracle.

Run once, in a container that has Hugging Face transformers installed (5.15.0 was used):

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py

The truth for every vector is the Hugging Face torch path of `Qwen3_5GatedDeltaNet`
(transformers/models/qwen3_5/modeling_qwen3_5.py): the layer the reference's own layer tests
compare against (wormhole_n150/qwen3.5_9B/test_gdn_layer.py:19-28,42-73 and
wormhole_n150/qwen3.5_0.8B/test_gdn_l1.py:31-52), and the recurrence that the reference's CPU oracle
restates (wormhole_n150/qwen3.5_9B/reference.py:1-2,11-35: "same math as HF
torch_recurrent_gated_delta_rule"). Nothing from the reference is imported or run here.

Input conventions follow the reference's tests:
  * layers: torch.manual_seed(seed), norm.weight ~ U(0.5, 1.5), dt_bias ~ U(-1, 1), projection
    weights rounded to bf16 (test_gdn_layer.py:19-28); x = randn(...).bfloat16().float() (:45);
  * recurrence: q, k, v, g = logsigmoid(randn + 2), beta = sigmoid(randn) drawn in that order from one
    torch.Generator (test_gated_delta_l1.py:17-24); initial state randn * 0.1 (:54).

Every file is a plain .npz of float32 arrays (no pickles) plus one JSON with the shapes and seeds.
"""

import json
import os
import sys

import numpy as np
import torch
import transformers
from transformers.cache_utils import DynamicCache
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

OUT = os.path.dirname(os.path.abspath(__file__))

TINY = dict(
    hidden_size=256, linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=32,
    linear_value_head_dim=32, linear_conv_kernel_dim=4, rms_norm_eps=1e-6, num_hidden_layers=4,
)


def f32(t):
    return np.ascontiguousarray(t.detach().float().cpu().numpy().astype(np.float32))


def make_layer(seed, cfg_kwargs):
    torch.manual_seed(seed)
    cfg = Qwen3_5TextConfig(**cfg_kwargs)
    layer = hf.Qwen3_5GatedDeltaNet(cfg, layer_idx=0).eval()
    with torch.no_grad():
        layer.norm.weight.uniform_(0.5, 1.5)
        layer.dt_bias.uniform_(-1.0, 1.0)
        for lin in (layer.in_proj_qkv, layer.in_proj_z, layer.in_proj_a, layer.in_proj_b, layer.out_proj):
            lin.weight.copy_(lin.weight.bfloat16().float())
    return cfg, layer


def layer_weights(layer):
    return {
        "w_qkv": f32(layer.in_proj_qkv.weight), "w_z": f32(layer.in_proj_z.weight),
        "w_a": f32(layer.in_proj_a.weight), "w_b": f32(layer.in_proj_b.weight),
        "conv_w": f32(layer.conv1d.weight[:, 0, :]), "A_log": f32(layer.A_log),
        "dt_bias": f32(layer.dt_bias), "norm_w": f32(layer.norm.weight), "w_out": f32(layer.out_proj.weight),
    }


def run_with_cache(cfg, layer, chunks):
    """Run the layer over consecutive chunks of x through one cache; returns (outputs, rec, conv[..., -3:])."""
    cache = DynamicCache(config=cfg)
    outs = []
    with torch.no_grad():
        for xc in chunks:
            outs.append(layer(xc, cache_params=cache))
    lay = cache.layers[0]
    return torch.cat(outs, 1), lay.recurrent_states[0], lay.conv_states[0][..., -3:]


def make_rec_inputs(B, T, Hk, Hv, dk, dv, seed, g_shift=2.0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hk, dk, generator=gen)
    k = torch.randn(B, T, Hk, dk, generator=gen)
    v = torch.randn(B, T, Hv, dv, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, Hv, generator=gen) + g_shift)
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=gen))
    return q, k, v, g, beta


def hf_recurrences(q, k, v, g, beta, init, chunk=64):
    """HF sequential and chunk-64 rules; q/k are repeat_interleaved to the v-heads as the layer does."""
    rep = v.shape[2] // q.shape[2]
    qr, kr = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
    with torch.no_grad():
        o_r, s_r = hf.torch_recurrent_gated_delta_rule(
            qr, kr, v, g=g, beta=beta, initial_state=init, output_final_state=True, use_qk_l2norm_in_kernel=True)
        o_c, s_c = hf.torch_chunk_gated_delta_rule(
            qr, kr, v, g=g, beta=beta, chunk_size=chunk, initial_state=init, output_final_state=True,
            use_qk_l2norm_in_kernel=True)
    return o_r, s_r, o_c, s_c


def main():
    meta = {"transformers": transformers.__version__, "torch": torch.__version__, "files": {}}

    # ---- tiny layer: one weight set, the reference's (B, T) grid plus a chunk-boundary case ----------
    cfg, layer = make_layer(0, TINY)
    np.savez(os.path.join(OUT, "tiny_weights.npz"), **layer_weights(layer))
    meta["files"]["tiny_weights.npz"] = {"seed": 0, "dims": TINY}
    for i, (B, T) in enumerate([(1, 1), (1, 40), (4, 9), (2, 70)]):
        torch.manual_seed(100 + i)
        x = torch.randn(B, T, TINY["hidden_size"]).bfloat16().float()
        out, rec, conv = run_with_cache(cfg, layer, [x])
        with torch.no_grad():
            out_nocache = layer(x)
        name = f"tiny_layer_B{B}_T{T}.npz"
        np.savez(os.path.join(OUT, name), x=f32(x), out=f32(out), out_nocache=f32(out_nocache),
                 rec_state=f32(rec), conv_state=f32(conv))
        meta["files"][name] = {"x_seed": 100 + i, "B": B, "T": T}

    # ---- prefill 20 then 5 single-token decode calls (HF cached decode path) ------------------------
    cfg1, layer1 = make_layer(1, TINY)
    torch.manual_seed(200)
    x = torch.randn(1, 25, TINY["hidden_size"]).bfloat16().float()
    out, rec, conv = run_with_cache(cfg1, layer1, [x[:, :20]] + [x[:, t:t + 1] for t in range(20, 25)])
    with torch.no_grad():
        out_full = layer1(x)
    np.savez(os.path.join(OUT, "tiny_continue.npz"), x=f32(x), out=f32(out), out_full=f32(out_full),
             rec_state=f32(rec), conv_state=f32(conv), **layer_weights(layer1))
    meta["files"]["tiny_continue.npz"] = {"weights_seed": 1, "x_seed": 200, "prefill": 20, "decode_steps": 5}

    # ---- recurrence alone ------------------------------------------------------------------------------
    cases = {
        "rec_gqa.npz": dict(shape=(2, 45, 2, 4, 32, 32), seed=0, g_shift=2.0, init=True),
        "rec_real_dims.npz": dict(shape=(1, 3, 2, 4, 128, 128), seed=1, g_shift=2.0, init=True),
        "rec_slow_decay.npz": dict(shape=(1, 300, 1, 2, 32, 32), seed=3, g_shift=5.0, init=False),
        "rec_chunk_edge.npz": dict(shape=(1, 130, 2, 2, 16, 24), seed=5, g_shift=0.0, init=True),
    }
    for name, c in cases.items():
        B, T, Hk, Hv, dk, dv = c["shape"]
        q, k, v, g, beta = make_rec_inputs(B, T, Hk, Hv, dk, dv, c["seed"], c["g_shift"])
        init = torch.randn(B, Hv, dk, dv, generator=torch.Generator().manual_seed(c["seed"] + 1000)) * 0.1 \
            if c["init"] else None
        o_r, s_r, o_c, s_c = hf_recurrences(q, k, v, g, beta, init)
        arrs = dict(q=f32(q), k=f32(k), v=f32(v), g=f32(g), beta=f32(beta), o=f32(o_r), state=f32(s_r),
                    o_chunk=f32(o_c), state_chunk=f32(s_c))
        if init is not None:
            arrs["init"] = f32(init)
        np.savez(os.path.join(OUT, name), **arrs)
        meta["files"][name] = {"B_T_Hk_Hv_dk_dv": list(c["shape"]), "seed": c["seed"], "g_shift": c["g_shift"],
                               "init": c["init"]}

    # ---- causal conv1d + SiLU: full-sequence form and the cached single-step update --------------------
    gen = torch.Generator().manual_seed(7)
    C, T = 16, 6
    xc = torch.randn(1, C, T, generator=gen)
    wc = torch.randn(C, 4, generator=gen) * 0.5
    with torch.no_grad():
        full = hf.causal_conv1d_fn(xc, wc, None, activation="silu")
        state = torch.zeros(1, C, 4)
        state[..., 4 - 3:] = xc[..., :3]  # history = the first 3 inputs
        steps = []
        for t in range(3, T):
            steps.append(hf.causal_conv1d_update(xc[..., t:t + 1], state, wc, None, activation="silu"))
    np.savez(os.path.join(OUT, "conv.npz"), x=f32(xc), w=f32(wc), out_full=f32(full),
             out_steps=f32(torch.cat(steps, -1)), state_after=f32(state[..., -3:]))
    meta["files"]["conv.npz"] = {"seed": 7, "C": C, "T": T}

    # ---- gated RMSNorm -------------------------------------------------------------------------------
    gen = torch.Generator().manual_seed(8)
    norm = hf.Qwen3_5RMSNormGated(32, eps=1e-6)
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5, generator=gen)
        o = torch.randn(10, 32, generator=gen) * 3.0
        z = torch.randn(10, 32, generator=gen)
        y = norm(o, z)
    np.savez(os.path.join(OUT, "rmsnorm_gated.npz"), o=f32(o), z=f32(z), w=f32(norm.weight), y=f32(y))
    meta["files"]["rmsnorm_gated.npz"] = {"seed": 8, "rows": 10, "dv": 32, "eps": 1e-6}

    with open(os.path.join(OUT, "golden_meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    total = sum(os.path.getsize(os.path.join(OUT, n)) for n in meta["files"])
    print(f"wrote {len(meta['files'])} fixtures, {total / 1e6:.2f} MB", file=sys.stderr)


if __name__ == "__main__":
    main()
