"""Recurrence-only gated delta rule on one MI355X: mirror of GatedDeltaRuleL1
(wormhole_n150/qwen3.5_9B/gated_delta_l1.py:131-272).

The recurrent state S[h] (dk x dv, fp32) of every (sequence, v-head) stays in device memory for the
lifetime of the object and is updated in place by each call, so consecutive calls continue the same
sequences (decode never moves the state to the host).  Inputs use the fla / HF layout:
q, k [B, T, Hk, dk], v [B, T, Hv, dv], g (log decay) and beta [B, T, Hv]; v-head h reads k-head
h // (Hv / Hk).  Per token (reference.py:28-34):  S = exp(g) S;  u = v - k^T S;  S = S + beta k u^T;
o = q^T S, with q, k L2-normalised and q scaled by dk ** -0.5.

Launches of more than 64 tokens with 128 x 128 heads run the chunk-64 form (HF's torch_chunk_gated_delta_rule,
HF:248-328: a parallel pass per 64-token chunk, then one sequential pass over the chunks) in a workspace the
object keeps on the device; `chunked=False` keeps every launch on the token loop.
"""

import ctypes

import torch

from . import _lib


class GatedDeltaRuleHIP:
    def __init__(self, num_heads, head_k_dim=128, head_v_dim=128, initial_state=None, device="cuda", chunked=True):
        """num_heads = B * Hv state tiles, as the reference's constructor takes them."""
        self.device = torch.device(device)
        self.num_heads = num_heads
        self.dk, self.dv = head_k_dim, head_v_dim
        self.chunked = chunked
        self.workspace = None  # uint8 device buffer of the chunked form, grown on demand
        self.state = torch.zeros(num_heads, head_k_dim, head_v_dim, device=self.device)
        self.reset_state(initial_state)

    def reset_state(self, initial_state=None):
        """Zero the state, or load `initial_state` [num_heads, dk, dv] (9B/gated_delta_l1.py:156-173).
        The buffer is reused, so its address never changes."""
        if initial_state is None:
            self.state.zero_()
        else:
            self.state.copy_(initial_state.reshape(self.num_heads, self.dk, self.dv))

    def get_state(self):
        """[num_heads, dk, dv] fp32 copy (9B/gated_delta_l1.py:175-177)."""
        return self.state.clone()

    def __call__(self, q, k, v, g, beta, use_qk_l2norm=True, scale=None):
        """Run T tokens for B sequences; returns o [B, T, Hv, dv] fp32 and updates the state."""
        B, T, Hk, dk = q.shape
        Hv, dv = v.shape[2], v.shape[3]
        if B * Hv != self.num_heads or dk != self.dk or dv != self.dv:
            raise ValueError(f"inputs B={B} Hv={Hv} dk={dk} dv={dv} do not match {self.num_heads} heads of "
                             f"{self.dk}x{self.dv}")
        dev = self.device
        t = [x.to(device=dev, dtype=torch.float32).contiguous() for x in (q, k, v, g, beta)]
        o = torch.empty(B, T, Hv, dv, device=dev)
        L = _lib.lib()
        need = L.gdn_delta_rule_fla_workspace_size(B, T, Hv, dk, dv) if self.chunked else 0
        if need and (self.workspace is None or self.workspace.numel() < need):
            self.workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        ws = self.workspace if need else None
        _lib.check(L.gdn_delta_rule_fla_ws(
            *[ctypes.c_void_p(x.data_ptr()) for x in t], B, T, Hk, Hv, dk, dv, ctypes.c_void_p(self.state.data_ptr()),
            int(bool(use_qk_l2norm)), float(scale or 0.0), ctypes.c_void_p(o.data_ptr()),
            ctypes.c_void_p(ws.data_ptr() if ws is not None else None), ws.numel() if ws is not None else 0,
            ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        return o
