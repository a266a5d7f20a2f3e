"""Local-checkpoint loader (linear_attention_op_amd/checkpoint.py) on synthetic safetensors files written here
with transformers' Qwen3.5 parameter names (modeling_qwen3_5.py:403-429): single file, sharded with an
index, the multimodal prefix, dims from shapes and config.json, and the error cases."""
import json
import os

import pytest
import torch
from safetensors.torch import save_file

from linear_attention_op_amd import synthetic as syn
from linear_attention_op_amd.checkpoint import linear_attention_layers, load_gdn_weights

NAMES = {"w_qkv": "in_proj_qkv.weight", "w_z": "in_proj_z.weight", "w_a": "in_proj_a.weight",
         "w_b": "in_proj_b.weight", "conv_w": "conv1d.weight", "A_log": "A_log", "dt_bias": "dt_bias",
         "norm_w": "norm.weight", "w_out": "out_proj.weight"}


def hf_tensors(w, prefix, i):
    out = {}
    for k, n in NAMES.items():
        t = w[k].bfloat16() if k in ("w_qkv", "w_z", "w_a", "w_b", "w_out") else w[k].float()
        if k == "conv_w":
            t = t[:, None, :].contiguous()
        out[f"{prefix}layers.{i}.linear_attn.{n}"] = t.contiguous()
    return out


def layers(d, n, seed=7):
    gen = torch.Generator().manual_seed(seed)
    return [syn.make_weights(d, seed=None, gen=gen)[0] for _ in range(n)]


def check_same(w_loaded, w_ref):
    for k in NAMES:
        ref = w_ref[k].bfloat16().float() if k in ("w_qkv", "w_z", "w_a", "w_b", "w_out") else w_ref[k].float()
        assert torch.equal(w_loaded[k].float(), ref), k


def test_sharded_directory_with_config(tmp_path):
    d = syn.SHAPES["tiny"]
    ws = layers(d, 2)
    t0 = hf_tensors(ws[0], "model.", 0)
    t2 = hf_tensors(ws[1], "model.", 2)
    t2["model.layers.1.self_attn.q_proj.weight"] = torch.zeros(4, 4)  # a full-attention layer in between
    save_file(t0, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(t2, str(tmp_path / "model-00002-of-00002.safetensors"))
    wm = {k: "model-00001-of-00002.safetensors" for k in t0}
    wm.update({k: "model-00002-of-00002.safetensors" for k in t2})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    (tmp_path / "config.json").write_text(json.dumps({
        "linear_key_head_dim": d["head_k_dim"], "linear_num_key_heads": d["num_k_heads"], "rms_norm_eps": 1e-5}))
    assert linear_attention_layers(str(tmp_path)) == [0, 2]
    dims, w = load_gdn_weights(str(tmp_path), 2)
    assert dims == dict(d, rms_norm_eps=1e-5)
    assert w["conv_w"].shape == (syn.conv_dim(d), 4)
    check_same(w, ws[1])
    with pytest.raises(KeyError):
        load_gdn_weights(str(tmp_path), 1)


def test_single_file_multimodal_prefix_without_config(tmp_path):
    d = syn.SHAPES["0.8b"]  # head_k_dim == head_v_dim, so the split follows from the shapes alone
    w = layers(d, 1)[0]
    f = tmp_path / "ckpt.safetensors"
    save_file(hf_tensors(w, "model.language_model.", 5), str(f))
    dims, wl = load_gdn_weights(str(f), 5)
    assert dims == d
    check_same(wl, w)
    assert linear_attention_layers(str(f)) == [5]


def test_errors(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_gdn_weights("Qwen/Qwen3.5-9B", 0)  # a hub name is not a path
    with pytest.raises(FileNotFoundError):
        load_gdn_weights(str(tmp_path), 0)      # a directory without a checkpoint
