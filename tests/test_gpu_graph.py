"""A decode step captured into a HIP graph replays exactly like eager launches.

The counterpart of the reference's traced decode (wormhole_n150/qwen3.5_0.8B/bench_decode.py:44-60,
gdn_l1.py:309-325).  Two layers with the same weights and initial state: one runs eagerly, the other is
captured once and replayed; between replays the test does its own eager work (new input copied into the
graph's static input, state read-back) and synchronises, and every replay is checked against the eager
step, output and recurrent state, bit for bit.
"""
import pytest
import torch

from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
from linear_attention_op_amd import synthetic as syn

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]


@pytest.mark.parametrize("shape, B", [("0.8b", 4), ("9b", 8)])
def test_graph_replay_matches_eager(shape, B):
    print(f"graph replay {shape} B={B}", flush=True)
    d = syn.SHAPES[shape]
    w, gen = syn.make_weights(d, seed=31)
    steps = 6
    x, s0 = syn.make_inputs(d, B, steps, gen, state_std=0.01)
    x = x.cuda().to(torch.bfloat16)
    eager = Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, max_tokens=64)
    graphed = Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, max_tokens=64)
    eager.set_state(rec=s0.cuda())
    graphed.set_state(rec=s0.cuda())
    torch.cuda.synchronize()

    x_static = x[:, 0:1].clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_static = graphed(x_static)
    torch.cuda.synchronize()
    # capture records the launches without running them: the graphed layer's state is still s0
    assert torch.equal(graphed.get_recurrent_state(), eager.get_recurrent_state())

    for t in range(steps):
        x_static.copy_(x[:, t:t + 1])
        g.replay()
        want = eager(x[:, t:t + 1])
        torch.cuda.synchronize()
        assert torch.equal(out_static, want), f"step {t}"
        assert torch.equal(graphed.get_recurrent_state(), eager.get_recurrent_state()), f"step {t}"
        torch.cuda.synchronize()
    assert torch.equal(graphed.get_conv_state(), eager.get_conv_state())
