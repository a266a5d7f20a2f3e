"""The C host driver of the ABI (csrc/gdn_driver.c) on the GPU: layer creation from host weights, a prefill,
decode steps timed on a HIP stream, the fp32 and bf16 outputs of one step equal to bf16 rounding, finite
outputs and states, state buffers in place, the error codes -- with no Python between the caller and the
library."""
import os
import subprocess

import pytest
import torch

from linear_attention_op_amd import _lib

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

EXE = os.path.join(os.path.dirname(_lib.LIB_PATH), "gdn_driver")


@pytest.mark.parametrize("args", [
    ["--shape", "0.8b", "--batch", "4", "--steps", "50", "--prefill", "200"],
    ["--shape", "9b", "--batch", "64", "--steps", "100", "--prefill", "1024"],
    ["--shape", "9b", "--batch", "8", "--steps", "50", "--prefill", "300", "--weights", "mxint8"],
])
def test_c_driver(args):
    print("gdn_driver", " ".join(args), flush=True)
    assert os.path.exists(EXE), "gdn_driver not built"
    r = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=240)
    print(r.stdout.strip(), r.stderr.strip(), flush=True)
    assert r.returncode == 0, r.stderr
    kv = dict(f.split("=", 1) for f in r.stdout.split())
    assert kv["checks_failed"] == "0"
    assert float(kv["decode_us_per_step"]) > 0
