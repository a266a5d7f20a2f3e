"""fp32 torch-CPU restatement of the reference's CPU path for the Gated DeltaNet layer.

Test infrastructure and the CPU baseline of bench.py only: nothing in the product imports it.

The reference's CPU path is pure PyTorch in fp32: the sequential recurrence of
wormhole_n150/qwen3.5_9B/reference.py:11-35 and, for the rest of the layer, the HF Qwen3_5GatedDeltaNet torch
fallbacks its tests treat as truth (9B/test_gdn_layer.py:19-28; transformers models/qwen3_5/
modeling_qwen3_5.py: causal conv 199-245, chunk-64 rule 248-328, gated RMSNorm 167-184, forward 432-543).
This module restates those algorithms with ATen operations so that the baseline runs at the speed of the
host's BLAS and threads, not of a naive loop:
  * projections: one fp32 GEMM over [W_qkv; W_z; W_a; W_b] and one over W_out (x @ W^T);
  * decode: one token per call for a batch, the per-token update of reference.py:28-34 batched over
    sequences and heads (S <- e^g S; u = beta (v - S^T k); S <- S + k u^T; o = S^T q);
  * prefill: the chunk-64 WY form of HF:248-328 for one sequence, chunk after chunk, batched over heads
    (T = (I + L)^-1 by a triangular solve).
State layout as the library's boundary: rec [B, nv, dk, dv] (S[k][v]), conv history [B, conv_dim, 3] in
time order (entry 2 newest).  It is checked against the fp64 oracle in tests/test_torch_ref.py.
"""

import math

import torch
import torch.nn.functional as F


class GDNLayerTorchCPU:
    """One layer on the CPU in fp32.  `w`: dict of tensors (w_qkv, w_z, w_a, w_b, conv_w [conv_dim, 4], A_log,
    dt_bias, norm_w, w_out), `d`: dims dict (hidden, num_k_heads, num_v_heads, head_k_dim, head_v_dim)."""

    def __init__(self, w, d, eps=1e-6):
        f = lambda t: torch.as_tensor(t).detach().to("cpu", torch.float32).contiguous()  # noqa: E731
        self.H, self.nk, self.nv = d["hidden"], d["num_k_heads"], d["num_v_heads"]
        self.dk, self.dv = d["head_k_dim"], d["head_v_dim"]
        self.Kd, self.Vd = self.nk * self.dk, self.nv * self.dv
        self.C = 2 * self.Kd + self.Vd
        self.ratio = self.nv // self.nk
        self.eps = eps
        self.w_in = torch.cat([f(w["w_qkv"]), f(w["w_z"]), f(w["w_a"]), f(w["w_b"])]).contiguous()
        self.w_out = f(w["w_out"])
        self.conv_w = f(w["conv_w"]).reshape(self.C, 4)
        self.neg_A = -torch.exp(f(w["A_log"]))
        self.dt_bias = f(w["dt_bias"])
        self.norm_w = f(w["norm_w"])

    # ---- pieces shared by both paths ------------------------------------------------------------------
    def _project(self, x):
        P = x @ self.w_in.T
        C, Vd, nv = self.C, self.Vd, self.nv
        return P[:, :C], P[:, C:C + Vd], P[:, C + Vd:C + Vd + nv], P[:, C + Vd + nv:]

    def _front(self, c, a, b):
        """post-conv channels c [M, C] -> q, k [M, nv, dk] (l2-normalised, q scaled, repeated per v-head),
        v [M, nv, dv], g, beta [M, nv]."""
        M = c.shape[0]
        q = c[:, :self.Kd].reshape(M, self.nk, self.dk)
        k = c[:, self.Kd:2 * self.Kd].reshape(M, self.nk, self.dk)
        v = c[:, 2 * self.Kd:].reshape(M, self.nv, self.dv)
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) / math.sqrt(self.dk)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        if self.ratio > 1:  # v-head h reads k-head h // ratio (repeat_interleave, reference.py:21-23)
            q = q.repeat_interleave(self.ratio, dim=1)
            k = k.repeat_interleave(self.ratio, dim=1)
        g = self.neg_A * F.softplus(a + self.dt_bias)  # threshold 20, as torch's default
        beta = torch.sigmoid(b)
        return q, k, v, g, beta

    def _norm_out(self, o, z):
        """gated RMSNorm per head (HF:167-184) and out_proj; o [M, nv, dv], z [M, Vd]."""
        M = o.shape[0]
        y = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + self.eps) * self.norm_w
        y = y * F.silu(z.reshape(M, self.nv, self.dv))
        return y.reshape(M, self.Vd) @ self.w_out.T

    # ---- decode: one token per sequence ----------------------------------------------------------------
    def decode(self, x, rec, conv):
        """x [B, H] -> out [B, H]; rec [B, nv, dk, dv] and conv [B, conv_dim, 3] are advanced in place."""
        qkv, z, a, b = self._project(x)
        window = torch.cat([conv, qkv.unsqueeze(-1)], -1)                     # [B, C, 4]: t-3 .. t
        c = F.silu((window * self.conv_w).sum(-1))
        conv.copy_(window[..., 1:])
        q, k, v, g, beta = self._front(c, a, b)
        rec.mul_(torch.exp(g)[..., None, None])                               # S <- e^g S
        kS = (k.unsqueeze(-2) @ rec).squeeze(-2)                              # S^T k  [B, nv, dv]
        u = beta.unsqueeze(-1) * (v - kS)
        rec.add_(k.unsqueeze(-1) * u.unsqueeze(-2))                           # S <- S + k u^T
        o = (q.unsqueeze(-2) @ rec).squeeze(-2)                               # S^T q
        return self._norm_out(o, z)

    # ---- prefill: chunk-64 form over one sequence ------------------------------------------------------
    def prefill(self, x, rec, conv, chunk=64):
        """x [T, H] of one sequence -> out [T, H]; rec [nv, dk, dv] and conv [conv_dim, 3] advanced in place."""
        T = x.shape[0]
        qkv, z, a, b = self._project(x)
        xt = torch.cat([conv.T, qkv], 0)                                      # [3 + T, C]
        c = F.silu(xt[0:T] * self.conv_w[:, 0] + xt[1:T + 1] * self.conv_w[:, 1] +
                   xt[2:T + 2] * self.conv_w[:, 2] + xt[3:T + 3] * self.conv_w[:, 3])
        conv.copy_(xt[T:T + 3].T)
        q, k, v, g, beta = self._front(c, a, b)                              # [T, nv, *]
        q, k, v = q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)    # [nv, T, *]
        g, beta = g.T, beta.T                                                 # [nv, T]
        o = torch.empty(self.nv, T, self.dv)
        S = rec
        eye = torch.eye(chunk)
        for t0 in range(0, T, chunk):
            n = min(chunk, T - t0)
            qc, kc, vc = q[:, t0:t0 + n], k[:, t0:t0 + n], v[:, t0:t0 + n]
            G = torch.cumsum(g[:, t0:t0 + n], -1)                             # in-chunk cumulative log decay
            bc = beta[:, t0:t0 + n].unsqueeze(-1)
            gam = torch.exp(G.unsqueeze(-1) - G.unsqueeze(-2)).tril()         # Gam_ij = e^(G_i - G_j), i >= j
            L = ((bc * kc) @ kc.transpose(-1, -2) * gam).tril(-1)             # strict lower
            IL = eye[:n, :n] + L
            U = torch.linalg.solve_triangular(IL, bc * vc, upper=False)       # T (beta V)
            W = torch.linalg.solve_triangular(IL, bc * kc * torch.exp(G).unsqueeze(-1), upper=False)
            Vn = U - W @ S                                                    # [nv, n, dv]
            Aqk = (qc @ kc.transpose(-1, -2)) * gam                           # tril incl. diagonal
            o[:, t0:t0 + n] = (qc * torch.exp(G).unsqueeze(-1)) @ S + Aqk @ Vn
            gl = G[:, -1:]
            S.mul_(torch.exp(gl).unsqueeze(-1))
            S.add_((kc * torch.exp(gl - G).unsqueeze(-1)).transpose(-1, -2) @ Vn)
        return self._norm_out(o.transpose(0, 1).contiguous(), z)
