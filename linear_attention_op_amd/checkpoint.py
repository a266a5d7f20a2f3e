"""Local-checkpoint loader: GDN layer weights from Hugging Face safetensors files on disk.

Feeds the layer's own re-layout (gdn_layer_create, the counterpart of the reference's _prepare_weights,
wormhole_n150/qwen3.5_9B/gdn_layer.py:90-127) from a checkpoint *path* -- a `.safetensors` file, or a
directory holding `model.safetensors` or a sharded `model.safetensors.index.json` (and, optionally, the
model's `config.json`).  Nothing is fetched: a hub name is not a path and is refused.

Parameter names follow transformers' Qwen3.5 model (modeling_qwen3_5.py:403-429, 740-746):
`<prefix>layers.<i>.linear_attn.{in_proj_qkv, in_proj_z, in_proj_a, in_proj_b, out_proj}.weight`,
`.conv1d.weight` [conv_dim, 1, 4] (no bias), `.A_log`, `.dt_bias`, `.norm.weight`, with prefix `model.`
(text model) or `model.language_model.` (the multimodal checkpoint).  Tensors are read through
safetensors' memory map, one layer at a time.
"""

import json
import os

_PREFIXES = ("model.", "model.language_model.", "")
_PARAMS = {  # weight-dict key -> parameter name under the layer's linear_attn module
    "w_qkv": "in_proj_qkv.weight", "w_z": "in_proj_z.weight", "w_a": "in_proj_a.weight",
    "w_b": "in_proj_b.weight", "conv_w": "conv1d.weight", "A_log": "A_log", "dt_bias": "dt_bias",
    "norm_w": "norm.weight", "w_out": "out_proj.weight",
}


def _files(path):
    """{tensor name: file} of a checkpoint path, and the directory (for config.json)."""
    if os.path.isfile(path):
        from safetensors import safe_open

        with safe_open(path, framework="pt") as f:
            return {k: path for k in f.keys()}, os.path.dirname(path)
    if not os.path.isdir(path):
        raise FileNotFoundError(f"{path!r} is not a safetensors file or a checkpoint directory "
                                "(hub names are not fetched)")
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f)["weight_map"]
        return {k: os.path.join(path, v) for k, v in wm.items()}, path
    single = os.path.join(path, "model.safetensors")
    if os.path.exists(single):
        return _files(single)[0], path
    raise FileNotFoundError(f"no model.safetensors or model.safetensors.index.json in {path!r}")


def _config(directory):
    """The text config fields of config.json, if present (nested under text_config for the multimodal one)."""
    p = os.path.join(directory, "config.json") if directory else ""
    if not p or not os.path.exists(p):
        return {}
    with open(p) as f:
        cfg = json.load(f)
    return cfg.get("text_config", cfg)


def load_gdn_weights(path, layer_idx, prefix=None):
    """-> (dims, weights) of GDN layer `layer_idx` of a local checkpoint, in the form Qwen35GatedDeltaNetHIP and
    Qwen35GDNStackHIP take (weights: CPU tensors in HF layouts, conv_w squeezed to [conv_dim, 4]).

    dims come from the tensor shapes; the k-head split (num_k_heads x head_k_dim) and rms_norm_eps from
    config.json when it is there, else head_k_dim = head_v_dim and eps = 1e-6."""
    from safetensors import safe_open

    where, directory = _files(path)
    cands = [prefix] if prefix is not None else list(_PREFIXES)
    base = None
    for p in cands:
        if f"{p}layers.{layer_idx}.linear_attn.A_log" in where:
            base = f"{p}layers.{layer_idx}.linear_attn."
            break
    if base is None:
        raise KeyError(f"layer {layer_idx} has no linear_attn parameters in {path!r} (prefixes tried: {cands})")
    w = {}
    handles = {}
    try:
        for key, name in _PARAMS.items():
            full = base + name
            if full not in where:
                raise KeyError(f"{full} missing from {path!r}")
            fn = where[full]
            if fn not in handles:
                handles[fn] = safe_open(fn, framework="pt")
            w[key] = handles[fn].get_tensor(full)
    finally:
        handles.clear()
    if w["conv_w"].dim() == 3:
        w["conv_w"] = w["conv_w"][:, 0, :]
    nv, H = w["w_a"].shape
    dv = w["norm_w"].shape[0]
    Vd = w["w_z"].shape[0]
    if Vd != nv * dv:
        raise ValueError(f"in_proj_z rows {Vd} != num_v_heads {nv} x head_v_dim {dv}")
    Kd2 = w["w_qkv"].shape[0] - Vd
    cfg = _config(directory)
    dk = int(cfg.get("linear_key_head_dim", dv))
    nk = int(cfg.get("linear_num_key_heads", Kd2 // 2 // dk))
    if 2 * nk * dk != Kd2:
        raise ValueError(f"in_proj_qkv rows {Kd2 + Vd}: 2 x {nk} x {dk} + {Vd} expected")
    dims = dict(hidden=H, num_k_heads=nk, num_v_heads=nv, head_k_dim=dk, head_v_dim=dv,
                conv_kernel=int(w["conv_w"].shape[-1]), rms_norm_eps=float(cfg.get("rms_norm_eps", 1e-6)))
    return dims, w


def linear_attention_layers(path, prefix=None):
    """Indices of the layers that have GDN (linear attention) parameters, in order."""
    where, _ = _files(path)
    out = set()
    for k in where:
        for p in ([prefix] if prefix is not None else _PREFIXES):
            if k.startswith(f"{p}layers.") and k.endswith(".linear_attn.A_log"):
                i = k[len(f"{p}layers."):].split(".")[0]
                if i.isdigit():
                    out.add(int(i))
    return sorted(out)
