"""ctypes binding of libgdn_hip.so (the C ABI declared in include/gdn.h).

Loading fails loudly when the library is not built: there is no CPU fallback for any op.
"""

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgdn_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "gdn.h")

GDN_OK = 0
GDN_ERR_INVALID_ARG = -1
GDN_ERR_UNSUPPORTED = -2
GDN_ERR_SHAPE = -3
GDN_ERR_SLOT = -4
GDN_ERR_HIP = -5
GDN_ERR_OUT_OF_MEMORY = -6

# gdn_weight_format; Python names follow the reference's weight_dtype argument
GDN_WEIGHTS_BF16 = 0
GDN_WEIGHTS_FP8_E4M3 = 1
GDN_WEIGHTS_MXFP4 = 2
GDN_WEIGHTS_MXINT8 = 3
WEIGHT_FORMATS = {"bf16": GDN_WEIGHTS_BF16, "bfloat16": GDN_WEIGHTS_BF16, "fp8": GDN_WEIGHTS_FP8_E4M3,
                  "fp8_e4m3": GDN_WEIGHTS_FP8_E4M3, "mxfp4": GDN_WEIGHTS_MXFP4, "fp4": GDN_WEIGHTS_MXFP4,
                  "mxint8": GDN_WEIGHTS_MXINT8, "int8": GDN_WEIGHTS_MXINT8}
WEIGHT_NAMES = {GDN_WEIGHTS_BF16: "bf16", GDN_WEIGHTS_FP8_E4M3: "fp8", GDN_WEIGHTS_MXFP4: "mxfp4",
                GDN_WEIGHTS_MXINT8: "mxint8"}


GDN_OUT_BF16 = 0
GDN_OUT_FP32 = 1


_OUT_NAMES = {"fp32": GDN_OUT_FP32, "float32": GDN_OUT_FP32, "bf16": GDN_OUT_BF16, "bfloat16": GDN_OUT_BF16}


def out_dtype_code(dtype):
    """torch.float32 or "fp32" (the reference's layer and stack output), torch.bfloat16 or "bf16" -> a
    gdn_out_dtype."""
    import torch

    if isinstance(dtype, str) and dtype.lower() in _OUT_NAMES:
        return _OUT_NAMES[dtype.lower()]
    if dtype == torch.float32:
        return GDN_OUT_FP32
    if dtype == torch.bfloat16:
        return GDN_OUT_BF16
    raise ValueError(f"output dtype {dtype}: torch.float32 / 'fp32' or torch.bfloat16 / 'bf16'")


def out_torch_dtype(dtype):
    """The torch dtype of an output dtype name or torch dtype."""
    import torch

    return torch.float32 if out_dtype_code(dtype) == GDN_OUT_FP32 else torch.bfloat16


def weight_format(weight_dtype):
    """gdn_weight_format of a weight_dtype name ("bf16", "fp8", "mxfp4" or "mxint8")."""
    try:
        return WEIGHT_FORMATS[str(weight_dtype).lower()]
    except KeyError:
        raise ValueError(f"weight_dtype {weight_dtype!r}: expected one of {sorted(WEIGHT_FORMATS)}") from None


class GdnError(RuntimeError):
    """A gdn_* call returned a negative status."""

    def __init__(self, code, message):
        super().__init__(f"gdn error {code}: {message}")
        self.code = code


class GdnValueError(GdnError, ValueError):
    """Bad argument, shape, slot or unsupported geometry (the reference raises assert / ValueError)."""


class GdnDims(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("num_k_heads", ctypes.c_int), ("num_v_heads", ctypes.c_int),
                ("head_k_dim", ctypes.c_int), ("head_v_dim", ctypes.c_int), ("conv_kernel", ctypes.c_int),
                ("rms_norm_eps", ctypes.c_float)]


class GdnWeights(ctypes.Structure):
    _fields_ = [("in_proj_qkv", ctypes.c_void_p), ("in_proj_z", ctypes.c_void_p), ("in_proj_a", ctypes.c_void_p),
                ("in_proj_b", ctypes.c_void_p), ("conv1d", ctypes.c_void_p), ("A_log", ctypes.c_void_p),
                ("dt_bias", ctypes.c_void_p), ("norm_weight", ctypes.c_void_p), ("out_proj", ctypes.c_void_p)]


_V = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "gdn_layer_create": (_I, [ctypes.POINTER(GdnDims), ctypes.POINTER(GdnWeights), _I, _I, ctypes.POINTER(_V)]),
    "gdn_layer_create_ex": (_I, [ctypes.POINTER(GdnDims), ctypes.POINTER(GdnWeights), _I, _I, _I,
                                 ctypes.POINTER(_V)]),
    "gdn_layer_weight_format": (_I, [_V]),
    "gdn_layer_set_output_dtype": (_I, [_V, _I]),
    "gdn_layer_output_dtype": (_I, [_V]),
    "gdn_layer_destroy": (_I, [_V]),
    "gdn_layer_forward": (_I, [_V, _V, _I, _I, _V, _V, _V]),
    "gdn_layer_forward_varlen": (_I, [_V, _V, _I, ctypes.POINTER(_I), _V, _V, _V]),
    "gdn_stack_create": (_I, [ctypes.POINTER(GdnDims), ctypes.POINTER(GdnWeights), _I, _I,
                              ctypes.POINTER(ctypes.c_void_p), _I, _I, ctypes.POINTER(_V)]),
    "gdn_stack_create_ex": (_I, [ctypes.POINTER(GdnDims), ctypes.POINTER(GdnWeights), _I, _I,
                                 ctypes.POINTER(ctypes.c_void_p), _I, _I, _I, ctypes.POINTER(_V)]),
    "gdn_stack_destroy": (_I, [_V]),
    "gdn_stack_layer": (_I, [_V, _I, ctypes.POINTER(_V)]),
    "gdn_stack_set_output_dtype": (_I, [_V, _I]),
    "gdn_stack_forward": (_I, [_V, _V, _I, _I, _V, _I, _I, _V, _V]),
    "gdn_stack_forward_varlen": (_I, [_V, _V, _I, ctypes.POINTER(_I), _V, _I, _I, _V, _V]),
    "gdn_state_reset": (_I, [_V, _V, _I, _V]),
    "gdn_state_get": (_I, [_V, _V, _I, _V, _V, _V]),
    "gdn_state_set": (_I, [_V, _V, _I, _V, _V, _V]),
    "gdn_layer_state_buffers": (_I, [_V, ctypes.POINTER(_V), ctypes.POINTER(_V), ctypes.POINTER(_V)]),
    "gdn_layer_proj_width": (_I, [_V]),
    "gdn_layer_profile": (_I, [_V, _I]),
    "gdn_layer_profile_read": (_I, [_V, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "gdn_in_proj": (_I, [_V, _V, _I, _V, _V]),
    "gdn_conv_front": (_I, [_V, _V, _I, _I, _V, _V, _V, _V, _V, _V, _V]),
    "gdn_delta_rule": (_I, [_V, _V, _V, _V, _V, _V, _I, _I, _V, _V, _V]),
    "gdn_gated_rmsnorm": (_I, [_V, _V, _V, _I, _I, _V, _V]),
    "gdn_out_proj": (_I, [_V, _V, _I, _V, _V]),
    "gdn_delta_rule_fla": (_I, [_V, _V, _V, _V, _V, _I, _I, _I, _I, _I, _I, _V, _I, _F, _V, _V]),
    "gdn_delta_rule_fla_workspace_size": (_Z, [_I, _I, _I, _I, _I]),
    "gdn_delta_rule_fla_ws": (_I, [_V, _V, _V, _V, _V, _I, _I, _I, _I, _I, _I, _V, _I, _F, _V, _V, _Z, _V]),
    "gdn_delta_rule_fla_noalloc": (_I, [_V, _V, _V, _V, _V, _I, _I, _I, _I, _I, _I, _V, _I, _F, _V, _V]),
    "gdn_linear_bf16": (_I, [_V, _V, _I, _I, _I, _V, _I, _V]),
    "gdn_quantize_fp8": (_I, [_V, _I, _I, _V, _V, _V]),
    "gdn_quantize_mxfp4": (_I, [_V, _I, _I, _V, _V, _V]),
    "gdn_quantize_mxint8": (_I, [_V, _I, _I, _V, _V, _V]),
    "gdn_last_error": (ctypes.c_char_p, []),
    "gdn_version": (_I, []),
}

_lib = None


def header_symbols():
    """Function names declared in include/gdn.h."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(gdn_\w+)\s*\(", text, re.M)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m linear_attention_op_amd.build` "
                               "(the Gated DeltaNet ops have no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != GDN_OK:
        msg = lib().gdn_last_error().decode(errors="replace")
        cls = GdnValueError if rc in (GDN_ERR_INVALID_ARG, GDN_ERR_UNSUPPORTED, GDN_ERR_SHAPE, GDN_ERR_SLOT) \
            else GdnError
        raise cls(rc, msg)
    return rc
