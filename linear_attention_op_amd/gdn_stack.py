"""A stack of Qwen3.5 GDN layers on one MI355X: host-side mirror of the reference's stack object.

Mirrors Qwen35_08B_GDNStackL1 (wormhole_n150/qwen3.5_0.8B/gdn_l1.py:207-341): layers of one geometry,
each with its own weights and states, run back to back -- `stack(x)` is one step through every layer,
`stack(x, layers=[i])` runs layer i alone -- plus `reset_state()` and `get_recurrent_state(i)`.  The
stack lives in libgdn_hip.so (gdn_stack_*): one C call per step, the layers sharing one launch
workspace.  Beyond the reference: prefill as well as decode, state slots, variable-length launches
(`forward_varlen`, a continuous batch of prefills and decode streams), and the decoder RMSNorm between
layers (`inter_norm=True`, HF Qwen3_5RMSNorm, modeling_qwen3_5.py:720-734).
"""

import ctypes

import torch

from . import _lib
from .gdn_layer import Qwen35GatedDeltaNetHIP, _ptr, _slots, _stream, cu_seqlens_arg, prepare_weights


class Qwen35GDNStackHIP:
    """`layers`: HF Qwen3_5GatedDeltaNet modules or weight dicts (see Qwen35GatedDeltaNetHIP), one per layer.
    `norm_weights`: optional per-layer [H] weights of the RMSNorm after each layer (default 0, i.e. (1 + w) = 1).
    `weight_dtype`: "bf16", "fp8", "mxfp4" or "mxint8" for every layer (wormhole_n150/qwen3.5_0.8B/gdn_l1.py:79-80).
    `out_dtype`: element type of the stack's output, torch.float32 as the reference's (gdn_l1.py:336-339 returns
    fp32 rows) or torch.bfloat16; the activations between layers are bf16 either way."""

    def __init__(self, layers, dims=None, batch=1, max_slots=None, max_tokens=None, inter_norm=False,
                 norm_weights=None, device="cuda", weight_dtype="bf16", out_dtype=torch.float32):
        self.device = torch.device(device)
        self.batch = batch
        self.max_slots = max_slots or batch
        self.max_tokens = max_tokens or max(64, batch)
        prepared = [prepare_weights(L, dims, self.device) for L in layers]
        self.dims = prepared[0][0]
        if any(p[0] != self.dims for p in prepared):
            raise ValueError("stacked layers must share one geometry")
        self.hidden = self.dims["hidden"]
        self.n_layers = len(prepared)
        cw = (_lib.GdnWeights * self.n_layers)(*[p[2] for p in prepared])
        keep = []
        nw = None
        if norm_weights is not None:
            nw = (ctypes.c_void_p * self.n_layers)()
            for i, w in enumerate(norm_weights):
                if w is not None:
                    t = torch.as_tensor(w).to(self.device, torch.float32).contiguous()
                    keep.append(t)
                    nw[i] = t.data_ptr()
        self._h = ctypes.c_void_p()
        torch.cuda.synchronize(self.device)
        _lib.check(_lib.lib().gdn_stack_create_ex(ctypes.byref(prepared[0][1]), cw, self.n_layers, int(inter_norm),
                                                  nw, self.max_slots, self.max_tokens,
                                                  _lib.weight_format(weight_dtype), ctypes.byref(self._h)))
        _lib.check(_lib.lib().gdn_stack_set_output_dtype(self._h, _lib.out_dtype_code(out_dtype)))
        self.out_dtype = _lib.out_torch_dtype(out_dtype)
        self.layers = []
        for i in range(self.n_layers):
            h = ctypes.c_void_p()
            _lib.check(_lib.lib().gdn_stack_layer(self._h, i, ctypes.byref(h)))
            self.layers.append(Qwen35GatedDeltaNetHIP(None, dims=self.dims, batch=batch, max_slots=self.max_slots,
                                                      max_tokens=self.max_tokens, device=device, _handle=h,
                                                      out_dtype=out_dtype))

    @classmethod
    def from_checkpoint(cls, path, layers=None, prefix=None, **kwargs):
        """The GDN layers `layers` (default: every linear-attention layer, in order) of a local safetensors
        checkpoint, stacked."""
        from .checkpoint import linear_attention_layers, load_gdn_weights

        idx = linear_attention_layers(path, prefix) if layers is None else list(layers)
        loaded = [load_gdn_weights(path, i, prefix) for i in idx]
        return cls([w for _, w in loaded], dims=loaded[0][0], **kwargs)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            for L in self.layers:
                L.close()
            _lib.lib().gdn_stack_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _runs(layers, n):
        """Consecutive runs (first, count) of the layer list (None = every layer)."""
        idx = list(range(n)) if layers is None else [int(i) for i in layers]
        runs = []
        for i in idx:
            if not 0 <= i < n:
                raise ValueError(f"layer {i} of {n}")
            if runs and runs[-1][0] + runs[-1][1] == i:
                runs[-1][1] += 1
            else:
                runs.append([i, 1])
        return runs

    def _run_dtype(self, first, count):
        """Element type of the output of the C call over layers [first, first + count): the stack's output type
        when it runs the last layer, else bf16 (activations)."""
        return self.out_dtype if first + count == self.n_layers else torch.bfloat16

    def __call__(self, hidden_states, layers=None, slot_ids=None):
        """hidden_states [B, H] (one decode step) or [B, T, H] -> same shape, of out_dtype, through `layers`
        (default all) in order, continuing the states of slots `slot_ids` (default 0..B-1).  gdn_l1.py:330-341.
        A list that does not end with the last layer returns the bf16 activations after its last layer, widened
        to out_dtype."""
        shape = hidden_states.shape
        x = hidden_states.to(device=self.device, dtype=torch.bfloat16)
        if x.dim() == 2:
            x = x.unsqueeze(1)
        B, T, H = x.shape
        if H != self.hidden:
            raise ValueError(f"hidden {H} != {self.hidden}")
        x = x.contiguous()
        s = _slots(slot_ids, self.device, self.max_slots, unique=True)
        for first, count in self._runs(layers, self.n_layers):
            x = x.to(torch.bfloat16)  # the fp32 output of an earlier run that ended at the last layer
            out = torch.empty(x.shape, device=self.device, dtype=self._run_dtype(first, count))
            _lib.check(_lib.lib().gdn_stack_forward(self._h, _ptr(x), B, T, _ptr(s), first, count, _ptr(out),
                                                    _stream()))
            x = out
        return x.to(self.out_dtype).reshape(shape)

    def forward_varlen(self, x, cu_seqlens, slot_ids=None, layers=None):
        """x [total, H]: a continuous batch -- sequence i is rows cu_seqlens[i]..cu_seqlens[i+1] and continues
        slot slot_ids[i] (default i); prefills and single-token decode streams mix freely."""
        n = len(cu_seqlens) - 1
        x = x.to(device=self.device, dtype=torch.bfloat16).reshape(-1, self.hidden).contiguous()
        cu = cu_seqlens_arg(cu_seqlens, n)
        s = _slots(slot_ids, self.device, self.max_slots, unique=True)
        for first, count in self._runs(layers, self.n_layers):
            x = x.to(torch.bfloat16)
            out = torch.empty(x.shape, device=self.device, dtype=self._run_dtype(first, count))
            _lib.check(_lib.lib().gdn_stack_forward_varlen(self._h, _ptr(x), n, cu, _ptr(s), first, count,
                                                           _ptr(out), _stream()))
            x = out
        return x.to(self.out_dtype)

    def reset_state(self, slot_ids=None):
        """Zero every layer's states (gdn_l1.py:203-205)."""
        for L in self.layers:
            L.reset_state(slot_ids)

    def get_recurrent_state(self, i, slot_ids=None):
        """[n, nv, dk, dv] fp32 copy of layer i's recurrent states (gdn_l1.py:207-212)."""
        return self.layers[i].get_recurrent_state(slot_ids)
