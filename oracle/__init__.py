"""CPU oracle for the Gated DeltaNet layer (ctypes over oracle/libgdn_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the benchmark's CPU-baseline
leg, always as the checker, never as the thing measured or shipped.  The product path
(linear_attention_op_amd) never imports this package.

Each function is a restatement of the reference's algorithm in C with fp64 accumulation; the C source
cites the reference file:line it follows.  Arrays are float32 numpy arrays at this boundary.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgdn_oracle.so")
_lib = None


def build():
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class Dims(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("nk", ctypes.c_int), ("nv", ctypes.c_int), ("dk", ctypes.c_int),
                ("dv", ctypes.c_int), ("kconv", ctypes.c_int), ("eps", ctypes.c_float)]


_P = ctypes.POINTER(ctypes.c_float)
_I = ctypes.c_int


def _declare(L):
    L.orc_set_threads.argtypes = [_I]
    L.orc_get_threads.restype = _I
    L.orc_khead_of_vhead.argtypes = [_I, _I, _I]
    L.orc_khead_of_vhead.restype = _I
    L.orc_conv_src.argtypes = [_I, _I, _I]
    L.orc_conv_src.restype = _I
    L.orc_roll_src.argtypes = [_I, _I]
    L.orc_roll_src.restype = _I
    L.orc_row_to_bt.argtypes = [_I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]
    L.orc_linear.argtypes = [_P, _P, _I, _I, _I, _P]
    L.orc_conv1d_silu.argtypes = [_P, _I, _I, _I, _P, _P, _P]
    L.orc_recurrent_gated_delta_rule.argtypes = [_P] * 5 + [_I] * 6 + [_P, _I, ctypes.c_float, _P, _P]
    L.orc_chunk_gated_delta_rule.argtypes = [_P] * 5 + [_I] * 6 + [_P, _I, ctypes.c_float, _I, _P, _P]
    L.orc_gated_rmsnorm.argtypes = [_P, _P, _I, _I, _P, ctypes.c_float, _P]
    L.orc_layer_forward.argtypes = [ctypes.POINTER(Dims)] + [_P] * 10 + [_I, _I] + [_P] * 5
    L.orc_conv_front.argtypes = [ctypes.POINTER(Dims), _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P]
    L.orc_e4m3_value.argtypes = [_I]
    L.orc_e4m3_value.restype = ctypes.c_double
    L.orc_e4m3_encode.argtypes = [ctypes.c_float]
    L.orc_e4m3_encode.restype = _I
    L.orc_quantize_e4m3.argtypes = [_P, _I, _I, ctypes.c_void_p, _P]
    L.orc_e2m1_value.argtypes = [_I]
    L.orc_e2m1_value.restype = ctypes.c_double
    L.orc_e2m1_encode.argtypes = [ctypes.c_float]
    L.orc_e2m1_encode.restype = _I
    L.orc_mx_scale_code.argtypes = [ctypes.c_float]
    L.orc_mx_scale_code.restype = _I
    L.orc_quantize_mxfp4.argtypes = [_P, _I, _I, ctypes.c_void_p, ctypes.c_void_p]
    L.orc_mx_scale_code_emax.argtypes = [ctypes.c_float, _I]
    L.orc_mx_scale_code_emax.restype = _I
    L.orc_mxint8_encode.argtypes = [ctypes.c_double]
    L.orc_mxint8_encode.restype = _I
    L.orc_quantize_mxint8.argtypes = [_P, _I, _I, ctypes.c_void_p, ctypes.c_void_p]


def _f(a):
    """float32 C-contiguous view (copy if needed) and its pointer."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_P)


def _ptr(a):
    return a.ctypes.data_as(_P)


def set_threads(n):
    lib().orc_set_threads(int(n))


def get_threads():
    return lib().orc_get_threads()


# ---- integer rules ------------------------------------------------------------------------------
def khead_of_vhead(h, nv, nk):
    return lib().orc_khead_of_vhead(h, nv, nk)


def conv_src(t, s, T):
    return lib().orc_conv_src(t, s, T)


def roll_src(T, k):
    return lib().orc_roll_src(T, k)


def row_to_bt(m, T):
    b, t = _I(), _I()
    lib().orc_row_to_bt(m, T, ctypes.byref(b), ctypes.byref(t))
    return b.value, t.value


# ---- ops ----------------------------------------------------------------------------------------
def linear(x, w):
    """y = x @ w.T with fp64 accumulation; x [M, K], w [N, K]."""
    x, px = _f(x)
    w, pw = _f(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_linear(px, pw, M, N, K, _ptr(y))
    return y


def conv1d_silu(x, w, hist):
    """x [B, T, C], w [C, 4], hist [B, C, 3] (time order) -> (out [B, T, C], new hist)."""
    x, px = _f(x)
    w, pw = _f(w)
    h = np.array(hist, dtype=np.float32, copy=True, order="C")
    B, T, C = x.shape
    out = np.empty_like(x)
    lib().orc_conv1d_silu(px, B, T, C, pw, _ptr(h), _ptr(out))
    return out, h


def recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None, use_qk_l2norm=True, scale=None):
    """Sequential gated delta rule; shapes as the reference: q, k [B,T,Hk,dk], v [B,T,Hv,dv], g, beta [B,T,Hv].
    Returns (o [B,T,Hv,dv], final_state [B,Hv,dk,dv])."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    g, pg = _f(g)
    beta, pb = _f(beta)
    B, T, Hk, dk = q.shape
    Hv, dv = v.shape[2], v.shape[3]
    o = np.empty((B, T, Hv, dv), np.float32)
    s = np.empty((B, Hv, dk, dv), np.float32)
    init = None
    if initial_state is not None:
        init, pi = _f(np.asarray(initial_state).reshape(B, Hv, dk, dv))
    lib().orc_recurrent_gated_delta_rule(pq, pk, pv, pg, pb, B, T, Hk, Hv, dk, dv,
                                         pi if init is not None else None, int(use_qk_l2norm),
                                         float(scale or 0.0), _ptr(o), _ptr(s))
    return o, s


def chunk_gated_delta_rule(q, k, v, g, beta, initial_state=None, use_qk_l2norm=True, scale=None, chunk=64):
    """Chunked (WY/UT) gated delta rule, same contract as recurrent_gated_delta_rule."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    g, pg = _f(g)
    beta, pb = _f(beta)
    B, T, Hk, dk = q.shape
    Hv, dv = v.shape[2], v.shape[3]
    o = np.empty((B, T, Hv, dv), np.float32)
    s = np.empty((B, Hv, dk, dv), np.float32)
    init = None
    if initial_state is not None:
        init, pi = _f(np.asarray(initial_state).reshape(B, Hv, dk, dv))
    lib().orc_chunk_gated_delta_rule(pq, pk, pv, pg, pb, B, T, Hk, Hv, dk, dv,
                                     pi if init is not None else None, int(use_qk_l2norm),
                                     float(scale or 0.0), int(chunk), _ptr(o), _ptr(s))
    return o, s


def gated_rmsnorm(o, z, w, eps=1e-6):
    """o, z [rows, dv], w [dv] -> y [rows, dv]."""
    o, po = _f(o)
    z, pz = _f(z)
    w, pw = _f(w)
    rows, dv = o.shape
    y = np.empty_like(o)
    lib().orc_gated_rmsnorm(po, pz, rows, dv, pw, float(eps), _ptr(y))
    return y


def dims(hidden, nk, nv, dk, dv, kconv=4, eps=1e-6):
    return Dims(hidden, nk, nv, dk, dv, kconv, eps)


def layer_forward(dm, weights, x, rec_state, conv_state, taps=False):
    """One launch of the whole layer.  weights: dict of float32 arrays in HF layouts (w_qkv, w_z, w_a, w_b,
    conv_w [conv_dim, 4], A_log, dt_bias, norm_w, w_out); x [B, T, H]; rec_state [B, nv, dk, dv] and
    conv_state [B, conv_dim, 3] are updated in place (must be float32 C-contiguous).
    Returns out [B, T, H] (and (y, o) taps [B*T, nv*dv] when taps=True)."""
    x, px = _f(x)
    B, T, H = x.shape
    for s in (rec_state, conv_state):
        assert s.dtype == np.float32 and s.flags.c_contiguous
    ws = [_f(weights[n]) for n in ("w_qkv", "w_z", "w_a", "w_b", "conv_w", "A_log", "dt_bias", "norm_w", "w_out")]
    out = np.empty((B, T, H), np.float32)
    Vd = dm.nv * dm.dv
    y = np.empty((B * T, Vd), np.float32) if taps else None
    o = np.empty((B * T, Vd), np.float32) if taps else None
    lib().orc_layer_forward(ctypes.byref(dm), *[p for _, p in ws], px, B, T, _ptr(rec_state), _ptr(conv_state),
                            _ptr(out), _ptr(y) if taps else None, _ptr(o) if taps else None)
    return (out, y, o) if taps else out


def conv_front(dm, P, B, T, weights, conv_state):
    """Front end from a fused projection row P [B*T, conv_dim + Vd + 2nv]; conv_state [B, conv_dim, 3] in place.
    Returns (qn [M,nk,dk], kn [M,nk,dk], v [M,nv,dv], g [M,nv], beta [M,nv])."""
    P, pp = _f(P)
    M = B * T
    assert conv_state.dtype == np.float32 and conv_state.flags.c_contiguous
    qn = np.empty((M, dm.nk, dm.dk), np.float32)
    kn = np.empty((M, dm.nk, dm.dk), np.float32)
    v = np.empty((M, dm.nv, dm.dv), np.float32)
    g = np.empty((M, dm.nv), np.float32)
    beta = np.empty((M, dm.nv), np.float32)
    cw, pcw = _f(weights["conv_w"])
    al, pal = _f(weights["A_log"])
    dt, pdt = _f(weights["dt_bias"])
    lib().orc_conv_front(ctypes.byref(dm), pp, B, T, pcw, pal, pdt, _ptr(conv_state), _ptr(qn), _ptr(kn), _ptr(v),
                         _ptr(g), _ptr(beta))
    return qn, kn, v, g, beta


# ---- low-precision weights (E4M3, one scale per row) -------------------------------------------------
def e4m3_table():
    """float32 [256]: the value of every E4M3 code (NaN for 0x7f and 0xff)."""
    return np.array([lib().orc_e4m3_value(c) for c in range(256)], np.float32)


def e4m3_encode(v):
    """E4M3 code of one float (nearest, ties to even, saturating at +-448)."""
    return lib().orc_e4m3_encode(float(v))


def quantize_e4m3(w):
    """w [N, K] -> (codes uint8 [N, K], scale float32 [N]) with scale = max|w[n]| / 448."""
    w, pw = _f(w)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N, np.float32)
    lib().orc_quantize_e4m3(pw, N, K, q.ctypes.data_as(ctypes.c_void_p), _ptr(s))
    return q, s


def dequantize_e4m3(q, scale):
    """codes [N, K], scale [N] -> float32 [N, K] = value(code) * scale (the weights the FP8 path multiplies by)."""
    return e4m3_table()[np.asarray(q)] * np.asarray(scale, np.float32)[:, None]


# ---- low-precision weights (MXFP4: E2M1 values, one E8M0 scale per 32 along K) ------------------------
def e2m1_table():
    """float32 [16]: the value of every E2M1 code."""
    return np.array([lib().orc_e2m1_value(c) for c in range(16)], np.float32)


def e2m1_encode(v):
    """E2M1 code of one float (nearest, ties to even, saturating at +-6)."""
    return lib().orc_e2m1_encode(float(v))


def mx_scale_code(amax):
    """E8M0 exponent byte of the scale 2^(floor(log2 amax) - 2) of a block with largest magnitude amax."""
    return lib().orc_mx_scale_code(float(amax))


def quantize_mxfp4(w):
    """w [N, K] (K % 32 == 0) -> (codes uint8 [N, K], one E2M1 code per byte; scale codes uint8 [N, K / 32])."""
    w, pw = _f(w)
    N, K = w.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    q = np.empty((N, K), np.uint8)
    sc = np.empty((N, K // 32), np.uint8)
    lib().orc_quantize_mxfp4(pw, N, K, q.ctypes.data_as(ctypes.c_void_p), sc.ctypes.data_as(ctypes.c_void_p))
    return q, sc


def dequantize_mxfp4(q, sc):
    """codes [N, K], scale codes [N, K / 32] -> float32 [N, K] = value(code) * 2^(scale code - 127)."""
    scale = np.ldexp(np.float32(1.0), np.asarray(sc, np.int32) - 127).astype(np.float32)
    return e2m1_table()[np.asarray(q)] * np.repeat(scale, 32, axis=1)


# ---- low-precision weights (MXINT8: int8 codes worth code * 2^-6, one E8M0 scale per 32 along K) -------
def mxint8_scale_code(amax):
    """E8M0 exponent byte of the MXINT8 scale 2^floor(log2 amax) of a block with largest magnitude amax."""
    return lib().orc_mx_scale_code_emax(float(amax), 0)


def mxint8_encode(v):
    """MXINT8 code of one value already divided by its block scale (nearest code / 64, ties to even, saturated)."""
    return lib().orc_mxint8_encode(float(v))


def quantize_mxint8(w):
    """w [N, K] (K % 32 == 0) -> (codes int8 [N, K]; scale codes uint8 [N, K / 32])."""
    w, pw = _f(w)
    N, K = w.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    q = np.empty((N, K), np.int8)
    sc = np.empty((N, K // 32), np.uint8)
    lib().orc_quantize_mxint8(pw, N, K, q.ctypes.data_as(ctypes.c_void_p), sc.ctypes.data_as(ctypes.c_void_p))
    return q, sc


def dequantize_mxint8(q, sc):
    """codes [N, K], scale codes [N, K / 32] -> float32 [N, K] = code * 2^(scale code - 133)."""
    step = np.ldexp(np.float64(1.0), np.asarray(sc, np.int32) - 133)
    return (np.asarray(q, np.float64) * np.repeat(step, 32, axis=1)).astype(np.float32)
