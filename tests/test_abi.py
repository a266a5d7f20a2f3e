"""The C-ABI library loads, exports every entry point include/gdn.h declares, and rejects bad arguments
on the host before touching a GPU (these calls return before any HIP launch or allocation)."""
import ctypes

import pytest

from linear_attention_op_amd import _lib


def test_header_declares_the_bound_entry_points():
    declared = _lib.header_symbols()
    assert set(declared) == set(_lib.SIGNATURES), (sorted(set(declared) ^ set(_lib.SIGNATURES)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in _lib.header_symbols():
        assert hasattr(L, name), name
    assert L.gdn_version() >= 100


def _dims(**kw):
    d = dict(hidden=1024, num_k_heads=16, num_v_heads=16, head_k_dim=128, head_v_dim=128, conv_kernel=4,
             rms_norm_eps=1e-6)
    d.update(kw)
    return _lib.GdnDims(*d.values())


@pytest.mark.parametrize("kw, code", [
    (dict(head_k_dim=96, head_v_dim=96), _lib.GDN_ERR_UNSUPPORTED),
    (dict(head_v_dim=64), _lib.GDN_ERR_UNSUPPORTED),
    (dict(num_v_heads=24), _lib.GDN_ERR_UNSUPPORTED),
    (dict(conv_kernel=3), _lib.GDN_ERR_UNSUPPORTED),
    (dict(hidden=1000), _lib.GDN_ERR_UNSUPPORTED),
    (dict(hidden=0), _lib.GDN_ERR_INVALID_ARG),
    # the fused mixer runs a k-head and its v-heads in one workgroup: at most 4 v-heads per k-head
    (dict(num_k_heads=4, num_v_heads=32), _lib.GDN_ERR_UNSUPPORTED),
])
def test_create_rejects_bad_geometry(kw, code):
    L = _lib.lib()
    h = ctypes.c_void_p()
    w = _lib.GdnWeights(*([1] * 9))  # never dereferenced: geometry is checked first
    rc = L.gdn_layer_create(ctypes.byref(_dims(**kw)), ctypes.byref(w), 1, 1, ctypes.byref(h))
    assert rc == code
    assert h.value is None
    assert L.gdn_last_error()


def test_null_arguments_are_errors_not_crashes():
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.gdn_layer_create(None, None, 1, 1, ctypes.byref(h)) == _lib.GDN_ERR_INVALID_ARG
    w = _lib.GdnWeights(*([0] * 9))
    assert L.gdn_layer_create(ctypes.byref(_dims()), ctypes.byref(w), 1, 1, ctypes.byref(h)) == \
        _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_layer_forward(None, None, 1, 1, None, None, None) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_state_get(None, None, 1, None, None, None) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_layer_destroy(None) == _lib.GDN_OK
    assert L.gdn_layer_set_output_dtype(None, _lib.GDN_OUT_FP32) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_layer_output_dtype(None) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_stack_set_output_dtype(None, _lib.GDN_OUT_BF16) == _lib.GDN_ERR_INVALID_ARG


def test_output_dtype_names():
    import torch

    assert _lib.out_dtype_code(torch.float32) == _lib.GDN_OUT_FP32 == 1
    assert _lib.out_dtype_code(torch.bfloat16) == _lib.GDN_OUT_BF16 == 0
    with pytest.raises(ValueError):
        _lib.out_dtype_code(torch.float16)


def test_linear_and_recurrence_shape_checks():
    L = _lib.lib()
    p = ctypes.c_void_p(16)  # non-null, never dereferenced
    assert L.gdn_linear_bf16(p, p, 4, 8, 100, p, 1, None) == _lib.GDN_ERR_UNSUPPORTED
    assert L.gdn_linear_bf16(p, p, 0, 8, 128, p, 1, None) == _lib.GDN_ERR_SHAPE
    args = [p] * 5
    assert L.gdn_delta_rule_fla(*args, 1, 1, 2, 3, 128, 128, p, 1, 0.0, p, None) == _lib.GDN_ERR_UNSUPPORTED
    assert L.gdn_delta_rule_fla(*args, 1, 1, 2, 4, 100, 100, p, 1, 0.0, p, None) == _lib.GDN_ERR_UNSUPPORTED
    assert L.gdn_delta_rule_fla(*args, 1, 0, 2, 4, 128, 128, p, 1, 0.0, p, None) == _lib.GDN_ERR_SHAPE


def test_chunked_recurrence_workspace_checks():
    L = _lib.lib()
    need = L.gdn_delta_rule_fla_workspace_size(2, 200, 32, 128, 128)
    # W, Q', keys (bf16 hi + lo) and U, the intra-chunk output, G (fp32) for 4 chunks of 64 tokens per (sequence, v-head)
    assert need == 2 * 32 * 4 * (64 * 128 * 3 + 64 * 128 * 2 + 64) * 4
    assert L.gdn_delta_rule_fla_workspace_size(2, 64, 32, 128, 128) == 0  # one chunk: the token loop
    assert L.gdn_delta_rule_fla_workspace_size(2, 200, 32, 64, 64) == 0   # chunked form is for 128 x 128
    assert L.gdn_delta_rule_fla_workspace_size(0, 200, 32, 128, 128) == 0
    p = ctypes.c_void_p(16)  # non-null, never dereferenced: the size is checked before any launch
    args = [p] * 5
    assert L.gdn_delta_rule_fla_ws(*args, 2, 200, 16, 32, 128, 128, p, 1, 0.0, p, p, need - 1, None) == \
        _lib.GDN_ERR_SHAPE
    assert b"workspace" in L.gdn_last_error()


def test_errors_raise_value_error_in_python():
    with pytest.raises(ValueError):
        _lib.check(_lib.GDN_ERR_SHAPE)
    with pytest.raises(_lib.GdnError):
        _lib.check(_lib.GDN_ERR_HIP)


def test_weight_format_checks():
    L = _lib.lib()
    h = ctypes.c_void_p()
    w = _lib.GdnWeights(*([1] * 9))  # never dereferenced: the format is checked before the weights
    assert L.gdn_layer_create_ex(ctypes.byref(_dims()), ctypes.byref(w), 1, 1, 7, ctypes.byref(h)) == \
        _lib.GDN_ERR_INVALID_ARG
    assert h.value is None and b"weight format" in L.gdn_last_error()
    assert L.gdn_stack_create_ex(ctypes.byref(_dims()), ctypes.byref(w), 2, 0, None, 1, 1, -1, ctypes.byref(h)) == \
        _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_layer_weight_format(None) == _lib.GDN_ERR_INVALID_ARG
    p = ctypes.c_void_p(16)
    assert L.gdn_quantize_fp8(None, 4, 64, p, p, None) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_quantize_fp8(p, 0, 64, p, p, None) == _lib.GDN_ERR_SHAPE
    assert _lib.weight_format("fp8") == _lib.GDN_WEIGHTS_FP8_E4M3 == _lib.weight_format("FP8_E4M3")
    assert _lib.weight_format("bf16") == _lib.GDN_WEIGHTS_BF16
    assert _lib.weight_format("mxfp4") == _lib.GDN_WEIGHTS_MXFP4 == _lib.weight_format("FP4")
    with pytest.raises(ValueError):
        _lib.weight_format("bfp4")
    # MXFP4: K a multiple of 32 for the quantizer
    assert L.gdn_quantize_mxfp4(None, 4, 64, p, p, None) == _lib.GDN_ERR_INVALID_ARG
    assert L.gdn_quantize_mxfp4(p, 0, 64, p, p, None) == _lib.GDN_ERR_SHAPE
    assert L.gdn_quantize_mxfp4(p, 4, 48, p, p, None) == _lib.GDN_ERR_UNSUPPORTED


def test_stack_rejects_inter_norm_wider_than_its_kernel():
    L = _lib.lib()
    h = ctypes.c_void_p()
    w = _lib.GdnWeights(*([1] * 9))  # never dereferenced: geometry is checked first
    rc = L.gdn_stack_create(ctypes.byref(_dims(hidden=8192 + 128)), ctypes.byref(w), 2, 1, None, 1, 1,
                            ctypes.byref(h))
    assert rc == _lib.GDN_ERR_UNSUPPORTED and b"RMSNorm" in L.gdn_last_error()
    assert h.value is None


def test_host_slot_ids_are_checked_before_upload():
    import torch

    from linear_attention_op_amd.gdn_layer import _slots

    cpu = torch.device("cpu")
    assert _slots(None, cpu, 4) is None
    assert _slots([3, 0, 2], cpu, 4, unique=True).tolist() == [3, 0, 2]
    for bad in ([0, 4], [-1], torch.tensor([1, 9])):
        with pytest.raises(_lib.GdnValueError) as e:
            _slots(bad, cpu, 4)
        assert e.value.code == _lib.GDN_ERR_SLOT
    with pytest.raises(_lib.GdnValueError):
        _slots([1, 1], cpu, 4, unique=True)
    assert _slots([1, 1], cpu, 4).tolist() == [1, 1]  # state reads may name a slot twice


def test_c_driver_links_and_parses_arguments():
    """The C host driver (csrc/gdn_driver.c, built beside the library) links against libgdn_hip.so and the HIP
    runtime and rejects a bad argument before it touches a device."""
    import os
    import subprocess

    exe = os.path.join(os.path.dirname(_lib.LIB_PATH), "gdn_driver")
    if not os.path.exists(exe):
        pytest.skip("gdn_driver not built (run __graft_entry__.build())")
    r = subprocess.run([exe, "--no-such-option"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage: gdn_driver" in r.stderr
    r = subprocess.run([exe, "--shape", "7b"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "shape 7b" in r.stderr
