"""Split-head decode against one workgroup per head, through the C ABI.

A single-token launch of at most 64 (sequence, v-head) pairs at 128-wide heads splits each head's state
over 4 workgroups of 32 columns. The gated RMSNorm then runs in the out_proj launch, from the mixer's
per-slice sums of squares, and that launch also advances the conv ring positions. A launch of more
sequences keeps one workgroup per head. Both run the same sequences here: the first Bs of a batch of
Bu > 64 / nv. The recurrence is the same arithmetic per state column with other partial-sum trees, so
states agree to fp32 rounding and outputs to the odd bf16 rounding of the normalised rows. The conv
history, read back in time order through the ring position, agrees bit for bit.
"""
import numpy as np
import pytest
import torch

from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
from linear_attention_op_amd import synthetic as syn

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]


def rel(a, b):
    a = np.asarray(a.float().cpu(), dtype=np.float64)
    b = np.asarray(b.float().cpu(), dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# (shape, split batch, whole batch): 9B has 32 v-heads (split up to batch 2), 0.8B 16 (up to batch 4)
@pytest.mark.parametrize("shape,Bs,Bu", [("9b", 1, 3), ("9b", 2, 3), ("0.8b", 1, 5), ("0.8b", 4, 5)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_split_head_decode_matches_per_head(shape, Bs, Bu, out_dtype):
    d = syn.SHAPES[shape]
    w, gen = syn.make_weights(d, seed=5)
    steps = 6
    x, s0 = syn.make_inputs(d, Bu, steps, gen, state_std=0.05)
    xp, _ = syn.make_inputs(d, Bu, 5, gen)
    split = Qwen35GatedDeltaNetHIP(w, dims=d, batch=Bs, max_tokens=64, out_dtype=out_dtype)
    whole = Qwen35GatedDeltaNetHIP(w, dims=d, batch=Bu, max_tokens=64, out_dtype=out_dtype)
    split.set_state(rec=s0[:Bs].cuda())
    whole.set_state(rec=s0.cuda())
    # a 5-token prefill first, so that the ring is full and its position is not 0 when the decode starts
    split(xp[:Bs])
    whole(xp)
    for t in range(steps):
        a = split(x[:Bs, t:t + 1])
        b = whole(x[:, t:t + 1])
        torch.cuda.synchronize()
        assert rel(a, b[:Bs]) < 1e-3, f"step {t}"
        assert rel(split.get_recurrent_state(), whole.get_recurrent_state()[:Bs]) < 1e-5, f"step {t}"
        assert torch.equal(split.get_conv_state().cpu(), whole.get_conv_state()[:Bs].cpu()), f"step {t}"


@pytest.mark.parametrize("weight_dtype", ["fp8", "mxfp4", "mxint8"])
def test_split_head_decode_low_precision_weights(weight_dtype):
    """The same comparison with E4M3 and MXFP4 weights (the out_proj's own GEMV block on the normalised rows
    in LDS), 9B at batch 1 against batch 3; MXINT8 keeps one workgroup per head at both batches."""
    d = syn.SHAPES["9b"]
    w, gen = syn.make_weights(d, seed=6)
    Bs, Bu, steps = 1, 3, 4
    x, s0 = syn.make_inputs(d, Bu, steps, gen, state_std=0.05)
    xp, _ = syn.make_inputs(d, Bu, 5, gen)
    split = Qwen35GatedDeltaNetHIP(w, dims=d, batch=Bs, max_tokens=64, weight_dtype=weight_dtype,
                                   out_dtype=torch.float32)
    whole = Qwen35GatedDeltaNetHIP(w, dims=d, batch=Bu, max_tokens=64, weight_dtype=weight_dtype,
                                   out_dtype=torch.float32)
    split.set_state(rec=s0[:Bs].cuda())
    whole.set_state(rec=s0.cuda())
    split(xp[:Bs])
    whole(xp)
    for t in range(steps):
        a = split(x[:Bs, t:t + 1])
        b = whole(x[:, t:t + 1])
        torch.cuda.synchronize()
        assert rel(a, b[:Bs]) < 1e-3, f"step {t}"
        assert rel(split.get_recurrent_state(), whole.get_recurrent_state()[:Bs]) < 1e-5, f"step {t}"
        assert torch.equal(split.get_conv_state().cpu(), whole.get_conv_state()[:Bs].cpu()), f"step {t}"
