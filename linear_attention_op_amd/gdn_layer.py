"""Qwen3.5 Gated DeltaNet layer on one MI355X: host-side mirror of the reference's layer object.

Mirrors Qwen35GatedDeltaNetTT (wormhole_n150/qwen3.5_9B/gdn_layer.py:54-292): built from an HF
`Qwen3_5GatedDeltaNet` (or a dict of its weights), it owns the weights, the per-sequence states and a
launch workspace; `layer(x)` runs x [B, T, H] -> [B, T, H] and continues every sequence from its
state; `reset_state()` / `get_recurrent_state()` as in the reference.  All compute runs in
libgdn_hip.so through its C ABI; torch only provides device memory and the stream.

Differences from the reference object, by design: state slots (a launch may name which slots its B
sequences use), bf16 activations at the boundary, and per-op entries for the five stages.
"""

import ctypes

import torch

from . import _lib

_WEIGHT_KEYS = ("w_qkv", "w_z", "w_a", "w_b", "conv_w", "A_log", "dt_bias", "norm_w", "w_out")


def weights_from_hf(layer):
    """HF Qwen3_5GatedDeltaNet -> (dims kwargs, weights dict of CPU tensors)."""
    dims = dict(hidden=layer.hidden_size, num_k_heads=layer.num_k_heads, num_v_heads=layer.num_v_heads,
                head_k_dim=layer.head_k_dim, head_v_dim=layer.head_v_dim, conv_kernel=layer.conv_kernel_size,
                rms_norm_eps=float(layer.layer_norm_epsilon))
    w = dict(w_qkv=layer.in_proj_qkv.weight, w_z=layer.in_proj_z.weight, w_a=layer.in_proj_a.weight,
             w_b=layer.in_proj_b.weight, conv_w=layer.conv1d.weight[:, 0, :], A_log=layer.A_log,
             dt_bias=layer.dt_bias, norm_w=layer.norm.weight, w_out=layer.out_proj.weight)
    return dims, {k: v.detach() for k, v in w.items()}


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _slots(slot_ids, device, max_slots=None, unique=False):
    """Slot ids as a device int32 tensor (None stays None).  Ids held on the host (lists, arrays, CPU tensors)
    are checked against [0, max_slots) -- and, for a launch (`unique`), for repeats -- before the upload; ids
    already on the device are passed through, and the kernels skip a sequence whose id is out of range
    (checking them here would synchronise)."""
    if slot_ids is None:
        return None
    on_device = isinstance(slot_ids, torch.Tensor) and slot_ids.device.type != "cpu"
    if not on_device and max_slots is not None:
        host = torch.as_tensor(slot_ids, dtype=torch.int64).reshape(-1)
        if host.numel() and (int(host.min()) < 0 or int(host.max()) >= max_slots):
            raise _lib.GdnValueError(_lib.GDN_ERR_SLOT,
                                     f"slot ids {host.tolist()} outside [0, {max_slots})")
        if unique and host.unique().numel() != host.numel():
            raise _lib.GdnValueError(_lib.GDN_ERR_SLOT, f"slot ids {host.tolist()} repeat a slot")
    s = torch.as_tensor(slot_ids, dtype=torch.int32, device=device).contiguous()
    return s


def prepare_weights(weights, dims, device):
    """(dims, C structs) for an HF layer or a weight dict: (dims dict, GdnDims, GdnWeights, tensors to keep
    alive until the create call returns)."""
    if hasattr(weights, "in_proj_qkv"):
        dims_hf, weights = weights_from_hf(weights)
        dims = dims or dims_hf
    if dims is None:
        raise ValueError("dims are required with a weight dict")
    missing = [k for k in _WEIGHT_KEYS if k not in weights]
    if missing:
        raise ValueError(f"missing weights: {missing}")
    d = dict(dims)

    def bf16(t):
        return torch.as_tensor(t).to(device=device, dtype=torch.bfloat16).contiguous()

    def f32(t):
        return torch.as_tensor(t).to(device=device, dtype=torch.float32).contiguous()

    w = {k: (bf16(weights[k]) if k in ("w_qkv", "w_z", "w_a", "w_b", "w_out") else f32(weights[k]))
         for k in _WEIGHT_KEYS}
    cdims = _lib.GdnDims(d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"],
                         d.get("conv_kernel", 4), d.get("rms_norm_eps", 1e-6))
    cw = _lib.GdnWeights(w["w_qkv"].data_ptr(), w["w_z"].data_ptr(), w["w_a"].data_ptr(), w["w_b"].data_ptr(),
                         w["conv_w"].data_ptr(), w["A_log"].data_ptr(), w["dt_bias"].data_ptr(),
                         w["norm_w"].data_ptr(), w["w_out"].data_ptr())
    return d, cdims, cw, w


def cu_seqlens_arg(cu_seqlens, n_seqs):
    """Host int32 array [n_seqs + 1] for the varlen entries."""
    cu = [int(v) for v in (cu_seqlens.tolist() if hasattr(cu_seqlens, "tolist") else cu_seqlens)]
    if len(cu) != n_seqs + 1:
        raise ValueError(f"cu_seqlens has {len(cu)} entries for {n_seqs} sequences")
    return (ctypes.c_int * len(cu))(*cu)


class Qwen35GatedDeltaNetHIP:
    """One GDN layer.  `weights` is an HF Qwen3_5GatedDeltaNet or a dict with keys
    w_qkv [conv_dim, H], w_z [Vd, H], w_a, w_b [nv, H], conv_w [conv_dim, 4], A_log, dt_bias [nv],
    norm_w [dv], w_out [H, Vd] (projection weights are used as bf16, the rest as fp32).
    `weight_dtype` ("bf16", "fp8", "mxfp4" or "mxint8") mirrors the reference's weight_dtype (9B/gdn_layer.py:55;
    bfloat8_b / bfloat4_b, 0.8B/gdn_l1.py:79-80): "fp8" keeps the q|k|v|z and out projections as E4M3 with
    per-row scales (see quantize_fp8), "mxfp4" as MXFP4 with a scale per 32 (see quantize_mxfp4), "mxint8" as
    MXINT8 with a scale per 32 (see quantize_mxint8; the bfloat8_b counterpart); a|b stay bf16.
    `out_dtype` is the element type of the layer's output: torch.float32, the reference's (9B/gdn_layer.py:272-276
    computes out_proj with dtype=ttnn.float32), or torch.bfloat16, the same sums rounded to nearest even."""

    def __init__(self, weights, dims=None, batch=1, max_slots=None, max_tokens=16384, device="cuda", _handle=None,
                 weight_dtype="bf16", out_dtype=torch.float32):
        self.device = torch.device(device)
        self.batch = batch
        self.max_slots = max_slots or batch
        self.max_tokens = max_tokens
        if _handle is not None:  # a layer owned by a stack
            self.dims = dict(dims)
            self._h, self._owned = _handle, False
        else:
            self.dims, cdims, cw, _keep = prepare_weights(weights, dims, self.device)
            self._h, self._owned = ctypes.c_void_p(), True
            torch.cuda.synchronize(self.device)
            _lib.check(_lib.lib().gdn_layer_create_ex(ctypes.byref(cdims), ctypes.byref(cw), self.max_slots,
                                                      self.max_tokens, _lib.weight_format(weight_dtype),
                                                      ctypes.byref(self._h)))
        d = self.dims
        self.hidden = d["hidden"]
        self.nk, self.nv = d["num_k_heads"], d["num_v_heads"]
        self.dk, self.dv = d["head_k_dim"], d["head_v_dim"]
        self.conv_dim = 2 * self.nk * self.dk + self.nv * self.dv
        self.proj_width = _lib.lib().gdn_layer_proj_width(self._h)
        fmt = _lib.lib().gdn_layer_weight_format(self._h)
        self.weight_dtype = _lib.WEIGHT_NAMES[fmt]
        _lib.check(_lib.lib().gdn_layer_set_output_dtype(self._h, _lib.out_dtype_code(out_dtype)))
        self.out_dtype = _lib.out_torch_dtype(out_dtype)

    @classmethod
    def from_checkpoint(cls, path, layer_idx, prefix=None, **kwargs):
        """Layer `layer_idx` of a local safetensors checkpoint (file or directory; see checkpoint.py)."""
        from .checkpoint import load_gdn_weights

        dims, w = load_gdn_weights(path, layer_idx, prefix)
        return cls(w, dims=dims, **kwargs)

    # ---- lifetime ---------------------------------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            if self._owned:
                _lib.lib().gdn_layer_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- layer ------------------------------------------------------------------------------------
    def __call__(self, hidden_states, slot_ids=None):
        """hidden_states [B, T, H] (any float dtype, used as bf16) -> [B, T, H] of out_dtype, continuing the
        states of slots `slot_ids` (default 0..B-1).  9B/gdn_layer.py:282-292."""
        B, T, H = hidden_states.shape
        if H != self.hidden:
            raise ValueError(f"hidden {H} != {self.hidden}")
        x = hidden_states.to(device=self.device, dtype=torch.bfloat16).contiguous()
        out = torch.empty(x.shape, device=self.device, dtype=self.out_dtype)
        s = _slots(slot_ids, self.device, self.max_slots, unique=True)
        _lib.check(_lib.lib().gdn_layer_forward(self._h, _ptr(x), B, T, _ptr(s), _ptr(out), _stream()))
        return out

    def forward_varlen(self, x, cu_seqlens, slot_ids=None):
        """x [total, H]: sequences of different lengths (rows cu_seqlens[i]..cu_seqlens[i+1]) in one launch,
        sequence i continuing slot slot_ids[i] (default i) -> [total, H] of out_dtype."""
        n = len(cu_seqlens) - 1
        x = x.to(device=self.device, dtype=torch.bfloat16).reshape(-1, self.hidden).contiguous()
        out = torch.empty(x.shape, device=self.device, dtype=self.out_dtype)
        s = _slots(slot_ids, self.device, self.max_slots, unique=True)
        _lib.check(_lib.lib().gdn_layer_forward_varlen(self._h, _ptr(x), n, cu_seqlens_arg(cu_seqlens, n), _ptr(s),
                                                       _ptr(out), _stream()))
        return out

    def reset_state(self, slot_ids=None):
        """Zero the conv and recurrent state of `slot_ids` (default: every slot).  9B/gdn_layer.py:137-151."""
        s = _slots(slot_ids, self.device, self.max_slots)
        n = self.max_slots if s is None else s.numel()
        _lib.check(_lib.lib().gdn_state_reset(self._h, _ptr(s), n, _stream()))

    def get_recurrent_state(self, slot_ids=None):
        """[n, nv, dk, dv] fp32 copy of the recurrent states (default: slots 0..batch-1).  9B/gdn_layer.py:153-157."""
        rec, _ = self.get_state(slot_ids, conv=False)
        return rec

    def get_conv_state(self, slot_ids=None):
        """[n, conv_dim, 3] fp32 conv history in time order (entry 2 = newest input)."""
        _, conv = self.get_state(slot_ids, rec=False)
        return conv

    def get_state(self, slot_ids=None, rec=True, conv=True):
        s = _slots(slot_ids, self.device, self.max_slots)
        n = self.batch if s is None else s.numel()
        r = torch.empty(n, self.nv, self.dk, self.dv, device=self.device) if rec else None
        c = torch.empty(n, self.conv_dim, 3, device=self.device) if conv else None
        _lib.check(_lib.lib().gdn_state_get(self._h, _ptr(s), n, _ptr(r), _ptr(c), _stream()))
        return r, c

    def set_state(self, rec=None, conv=None, slot_ids=None):
        """Seed slots with rec [n, nv, dk, dv] and conv [n, conv_dim, 3] (None conv = zero history)."""
        s = _slots(slot_ids, self.device, self.max_slots)
        ref = rec if rec is not None else conv
        n = ref.shape[0] if s is None else s.numel()
        r = rec.to(self.device, torch.float32).contiguous() if rec is not None else None
        c = conv.to(self.device, torch.float32).contiguous() if conv is not None else None
        _lib.check(_lib.lib().gdn_state_set(self._h, _ptr(s), n, _ptr(r), _ptr(c), _stream()))

    def state_buffers(self):
        """Device addresses (rec, conv, conv_pos) of the resident state buffers: the recurrent states, the conv
        history rings and their positions."""
        r, c, p = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(_lib.lib().gdn_layer_state_buffers(self._h, ctypes.byref(r), ctypes.byref(c), ctypes.byref(p)))
        return r.value, c.value, p.value

    def profile(self, max_calls):
        """Record stage times (HIP events on the launch stream) for the next `max_calls` forward calls."""
        _lib.check(_lib.lib().gdn_layer_profile(self._h, int(max_calls)))

    def profile_read(self):
        """-> (dict of summed ms per stage: in_proj, mixer, out_proj, total; number of calls recorded)."""
        ms = (ctypes.c_double * 4)()
        n = ctypes.c_int()
        _lib.check(_lib.lib().gdn_layer_profile_read(self._h, ms, ctypes.byref(n)))
        return dict(zip(("in_proj", "mixer", "out_proj", "total"), list(ms))), n.value

    # ---- per-op entries ---------------------------------------------------------------------------
    def in_proj(self, x):
        """x [M, H] -> P [M, proj_width] fp32 (q | k | v | z | a | b)."""
        x = x.to(device=self.device, dtype=torch.bfloat16).contiguous()
        P = torch.empty(x.shape[0], self.proj_width, device=self.device)
        _lib.check(_lib.lib().gdn_in_proj(self._h, _ptr(x), x.shape[0], _ptr(P), _stream()))
        return P

    def conv_front(self, P, B, T, slot_ids=None):
        """P [B*T, proj_width] -> (qn [M,nk,dk], kn [M,nk,dk], v [M,nv,dv], g [M,nv], beta [M,nv]);
        advances the conv history of the slots."""
        M = B * T
        dev = self.device
        qn = torch.empty(M, self.nk, self.dk, device=dev)
        kn = torch.empty(M, self.nk, self.dk, device=dev)
        v = torch.empty(M, self.nv, self.dv, device=dev)
        g = torch.empty(M, self.nv, device=dev)
        beta = torch.empty(M, self.nv, device=dev)
        s = _slots(slot_ids, dev, self.max_slots, unique=True)
        P = P.contiguous()
        _lib.check(_lib.lib().gdn_conv_front(self._h, _ptr(P), B, T, _ptr(s), _ptr(qn), _ptr(kn), _ptr(v), _ptr(g),
                                             _ptr(beta), _stream()))
        return qn, kn, v, g, beta

    def delta_rule(self, qn, kn, v, g, beta, B, T, slot_ids=None):
        """Recurrence on the front end's outputs, continuing the slots' states -> o [M, nv, dv] fp32."""
        o = torch.empty(B * T, self.nv, self.dv, device=self.device)
        s = _slots(slot_ids, self.device, self.max_slots, unique=True)
        t = [x.contiguous() for x in (qn, kn, v, g, beta)]
        _lib.check(_lib.lib().gdn_delta_rule(self._h, *[_ptr(x) for x in t], B, T, _ptr(s), _ptr(o), _stream()))
        return o

    def gated_rmsnorm(self, o, z):
        """o [M, nv*dv] fp32, z [M, >= nv*dv] fp32 rows -> y [M, nv*dv] bf16."""
        M = o.shape[0]
        o = o.reshape(M, -1).contiguous()
        y = torch.empty(M, self.nv * self.dv, device=self.device, dtype=torch.bfloat16)
        _lib.check(_lib.lib().gdn_gated_rmsnorm(self._h, _ptr(o), _ptr(z), z.stride(0), M, _ptr(y), _stream()))
        return y

    def out_proj(self, y):
        """y [M, nv*dv] -> out [M, H] of out_dtype."""
        y = y.to(device=self.device, dtype=torch.bfloat16).contiguous()
        out = torch.empty(y.shape[0], self.hidden, device=self.device, dtype=self.out_dtype)
        _lib.check(_lib.lib().gdn_out_proj(self._h, _ptr(y), y.shape[0], _ptr(out), _stream()))
        return out


def linear(x, w, out_dtype=torch.float32):
    """y = x @ w.T on the library's bf16 MFMA projection kernels (x [M, K], w [N, K], K % 128 == 0)."""
    x = x.to(torch.bfloat16).contiguous()
    w = w.to(torch.bfloat16).contiguous()
    y = torch.empty(x.shape[0], w.shape[0], device=x.device, dtype=out_dtype)
    _lib.check(_lib.lib().gdn_linear_bf16(_ptr(x), _ptr(w), x.shape[0], w.shape[0], x.shape[1], _ptr(y),
                                          int(out_dtype == torch.float32), _stream()))
    return y


def quantize_fp8(w):
    """The library's E4M3 weight quantizer (gdn_quantize_fp8) on a CUDA matrix w [N, K]: -> (codes uint8 [N, K],
    scales fp32 [N]); row n dequantizes to e4m3_value(codes[n]) * scales[n], scales[n] = max|w[n]| / 448."""
    w = w.to(torch.bfloat16).contiguous()
    q = torch.empty(w.shape, device=w.device, dtype=torch.uint8)
    s = torch.empty(w.shape[0], device=w.device, dtype=torch.float32)
    _lib.check(_lib.lib().gdn_quantize_fp8(_ptr(w), w.shape[0], w.shape[1], _ptr(q), _ptr(s), _stream()))
    return q, s


def quantize_mxfp4(w):
    """The library's MXFP4 weight quantizer (gdn_quantize_mxfp4) on a CUDA matrix w [N, K] (K % 32 == 0): ->
    (codes uint8 [N, K / 2], two E2M1 codes per byte, column 2i in the low nibble; scale codes uint8 [N, K / 32],
    E8M0).  Block j of row n dequantizes to e2m1_value(codes) * 2^(scale[n, j] - 127)."""
    w = w.to(torch.bfloat16).contiguous()
    N, K = w.shape
    q = torch.empty((N, K // 2), device=w.device, dtype=torch.uint8)
    s = torch.empty((N, K // 32), device=w.device, dtype=torch.uint8)
    _lib.check(_lib.lib().gdn_quantize_mxfp4(_ptr(w), N, K, _ptr(q), _ptr(s), _stream()))
    return q, s


def quantize_mxint8(w):
    """The library's MXINT8 weight quantizer (gdn_quantize_mxint8) on a CUDA matrix w [N, K] (K % 32 == 0): ->
    (codes int8 [N, K]; scale codes uint8 [N, K / 32], E8M0).  Block j of row n dequantizes to
    codes * 2^(scale[n, j] - 133)."""
    w = w.to(torch.bfloat16).contiguous()
    N, K = w.shape
    q = torch.empty((N, K), device=w.device, dtype=torch.int8)
    s = torch.empty((N, K // 32), device=w.device, dtype=torch.uint8)
    _lib.check(_lib.lib().gdn_quantize_mxint8(_ptr(w), N, K, _ptr(q), _ptr(s), _stream()))
    return q, s
