"""gdn_delta_rule_fla_noalloc (the recurrence-only op with its chunk workspace in a static device array)
against gdn_delta_rule_fla_ws with a caller-allocated workspace, through the C ABI: bit-exact outputs and
final states on two calls in a row, the second smaller than the first (the array keeps the first call's
contents), a token-loop call that needs no workspace, and the size limit checked before any launch."""
import ctypes

import pytest
import torch

from linear_attention_op_amd import _lib

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]


def _inputs(B, T, Hk, Hv, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    k = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    v = torch.randn(B, T, Hv, D, device="cuda", generator=g)
    gg = torch.nn.functional.logsigmoid(torch.randn(B, T, Hv, device="cuda", generator=g) + 2.0)
    beta = torch.sigmoid(torch.randn(B, T, Hv, device="cuda", generator=g))
    s0 = torch.randn(B, Hv, D, D, device="cuda", generator=g) * 0.01
    return q, k, v, gg, beta, s0


def _run(noalloc, B, T, Hk, Hv, D, seed):
    L = _lib.lib()
    q, k, v, g, beta, s0 = _inputs(B, T, Hk, Hv, D, seed)
    state = s0.clone()
    o = torch.empty(B, T, Hv, D, device="cuda")
    p = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, g, beta)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = L.gdn_delta_rule_fla_noalloc(*p, B, T, Hk, Hv, D, D, ctypes.c_void_p(state.data_ptr()), 1, 0.0,
                                          ctypes.c_void_p(o.data_ptr()), stream)
    else:
        need = L.gdn_delta_rule_fla_workspace_size(B, T, Hv, D, D)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
        rc = L.gdn_delta_rule_fla_ws(*p, B, T, Hk, Hv, D, D, ctypes.c_void_p(state.data_ptr()), 1, 0.0,
                                     ctypes.c_void_p(o.data_ptr()), ctypes.c_void_p(ws.data_ptr() if need else None),
                                     need, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return o, state


@pytest.mark.parametrize("shapes", [[(2, 300, 4, 8), (1, 130, 4, 8)],   # chunked twice, the second smaller
                                    [(3, 200, 2, 4), (1, 40, 2, 4)]])  # chunked, then the token loop
def test_noalloc_equals_workspace_entry(shapes):
    for i, (B, T, Hk, Hv) in enumerate(shapes):
        print(f"noalloc call {i}: B={B} T={T} Hk={Hk} Hv={Hv}", flush=True)
        o_n, s_n = _run(True, B, T, Hk, Hv, 128, seed=10 + i)
        o_w, s_w = _run(False, B, T, Hk, Hv, 128, seed=10 + i)
        assert torch.isfinite(o_n).all()
        assert torch.equal(o_n, o_w), f"call {i}: output"
        assert torch.equal(s_n, s_w), f"call {i}: final state"


def test_noalloc_rejects_launches_beyond_the_array():
    L = _lib.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the size is checked before any launch
    # one 16384-token sequence of 32 heads: 8192 head-chunks of workspace, the array holds 408
    rc = L.gdn_delta_rule_fla_noalloc(p, p, p, p, p, 1, 16384, 16, 32, 128, 128, p, 1, 0.0, p, None)
    assert rc == _lib.GDN_ERR_SHAPE
    assert b"static scratch" in L.gdn_last_error()
