"""Benchmark of the Qwen3.5-9B-shape Gated DeltaNet layer on one MI355X.

    python bench.py [--steps K] [--warmup W]

Headline (the `value` of the JSON line): decode throughput at batch 64 -- tokens per second through one
9B-shape GDN layer, one step = one token for each of the 64 sequences (in_proj -> fused mixer ->
out_proj), inputs and states resident in HBM.  To keep the 256 MB Infinity Cache from serving the
weights, the timed steps rotate over `--copies` independent layers (own weights, own 64 state slots;
> 1 GB working set), as consecutive layers of a model would.

Also reported: prefill of one 16384-token sequence (tokens/s and bf16-MFMA roofline fraction), the
roofline of the dominant decode kernel (the fused mixer, timed with HIP events on its stream), and the
CPU oracle timed on a bounded sample of the same decode workload on the host cores.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GDN-layer decode tok/s + prefill tok/s at 9B shape; % HBM / MFMA roofline"
HBM_PEAK = 8.0e12        # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15       # FLOP/s, MI355X dense bf16 MFMA
LAYER_OUT = "bf16"       # layer / stack output element type: bf16 activations, as in a bf16 model
# Every measured workload first runs untimed for SETTLE_S seconds, then its warm-up steps, then the timed
# steps.  From idle the clocks take tens of milliseconds to rise: the 16k prefill measured 3.33 ms per call
# after one warm-up call against 2.90-2.92 ms after 200 ms of calls (in_proj GEMM 1.64 -> 1.40 ms), the
# batch-64 decode 90 against 88-89 us per step.
SETTLE_S = 0.3


def settle(fn, seconds=SETTLE_S):
    """Run fn() untimed until `seconds` have passed, synchronising about every 20 ms; returns the call count."""
    import torch

    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    k = max(1, int(0.02 / max(time.perf_counter() - t0, 1e-6)))
    n = 1
    while time.perf_counter() - t0 < seconds:
        for _ in range(k):
            fn()
        n += k
        torch.cuda.synchronize()
    return n


def decode_bytes(d, B, weights="bf16"):
    """Algorithmic HBM bytes of one decode layer step: weights once plus per-sequence state and I/O.
    W = bf16 projections (qkv, z, a, b, out) + bf16 conv taps (fp8: qkv, z and out as 1-byte codes plus an
    fp32 scale per row; mxfp4: the same as half-byte codes plus a 1-byte scale per 32; mxint8: 1-byte codes
    plus a 1-byte scale per 32; a and b bf16); s = fp32 state read + write, fp32 conv history (3 reads + 1 write
    per channel), bf16 x in and out."""
    H, nk, nv, dk, dv = d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"]
    C, Vd = 2 * nk * dk + nv * dv, nv * dv
    q = C * H + Vd * H + H * Vd  # quantized weights
    if weights == "fp8":
        W = q + 4 * (C + Vd + H) + 2 * 2 * nv * H + 2 * C * 4
    elif weights == "mxfp4":
        W = q // 2 + q // 32 + 2 * 2 * nv * H + 2 * C * 4
    elif weights == "mxint8":
        W = q + q // 32 + 2 * 2 * nv * H + 2 * C * 4
    else:
        W = 2 * (C * H + Vd * H + 2 * nv * H + H * Vd) + 2 * C * 4
    s = nv * dk * dv * 4 * 2 + C * 4 * 4 + 2 * H * 2
    return W, s


def eager_decode(layers, xs, steps, warmup):
    """Wall ms per eager decode step over `layers` in rotation, and the per-stage HIP-event averages."""
    import torch

    L = len(layers)
    it = iter(range(1 << 62))
    settle(lambda: (lambda i: layers[i % L](xs[i % len(xs)]))(next(it)))
    for i in range(warmup):
        layers[i % L](xs[i % len(xs)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        layers[i % L](xs[i % len(xs)])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    for lay in layers:
        lay.profile(steps)
    for i in range(steps):
        layers[i % L](xs[i % len(xs)])
    torch.cuda.synchronize()
    stage = {"in_proj": 0.0, "mixer": 0.0, "out_proj": 0.0, "total": 0.0}
    calls = 0
    for lay in layers:
        ms, n = lay.profile_read()
        calls += n
        for k in stage:
            stage[k] += ms[k]
        lay.profile(0)
    return wall, {k: v / max(calls, 1) for k, v in stage.items()}


def mixer_bytes_per_seq(d):
    """Algorithmic bytes of the fused mixer kernel per sequence and token: fp32 state read + write,
    conv history (3 reads + 1 write, fp32), the fp32 projection row it consumes (q|k|v|z|a|b) and the
    bf16 normalised output row it writes."""
    nk, nv, dk, dv = d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"]
    C, Vd = 2 * nk * dk + nv * dv, nv * dv
    return nv * dk * dv * 4 * 2 + C * 4 * 4 + (C + Vd + 2 * nv) * 4 + Vd * 2


def prefill_flops_per_token(d, chunk=64):
    """Projections (in: q|k|v|z|a|b, out) plus the chunk-64 WY/UT form of the recurrence."""
    H, nk, nv, dk, dv = d["hidden"], d["num_k_heads"], d["num_v_heads"], d["head_k_dim"], d["head_v_dim"]
    Kd, Vd = nk * dk, nv * dv
    C = chunk
    proj = 2 * H * (2 * Kd + 2 * Vd + 2 * nv) + 2 * Vd * H
    rec = nv * (2 * C * (3 * dk + 2 * dv) + 6 * dk * dv + 2 * C * C / 3)
    return proj + rec


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, warmup=10, reps=20):
    """Median wall seconds of `reps` calls after `warmup` untimed ones (the reference's bench protocol,
    wormhole_n150/qwen3.5_0.8B/bench_decode.py:29-41)."""
    import statistics

    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(w9, prefill_prefix=256, oracle_seconds=2.0):
    """The reference's CPU path timed on this host: an fp32 torch restatement of it (oracle/torch_ref.py:
    ATen GEMMs, the per-token recurrence for decode, the chunk-64 form for prefill), with all the host threads
    the process may use, 10 warm-ups and the median of 20 runs per row.  Rows: 9B decode at batch 64 (the
    headline workload), 0.8B decode at batch 1, and the 9B 16k prefill extrapolated from a prefix.  The fp64
    oracle's rate on the headline workload is kept as a side figure."""
    import numpy as np
    import torch

    import oracle
    from linear_attention_op_amd import synthetic as syn
    from oracle.torch_ref import GDNLayerTorchCPU

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(2)
    rows = {}
    t_start = time.perf_counter()

    d9 = syn.SHAPES["9b"]
    lay = GDNLayerTorchCPU(w9, d9)
    B = 64
    x = torch.randn(B, d9["hidden"], generator=gen).bfloat16().float()
    rec = torch.randn(B, d9["num_v_heads"], 128, 128, generator=gen) * 0.01
    conv = torch.zeros(B, syn.conv_dim(d9), 3)
    t = _median_time(lambda: lay.decode(x, rec, conv))
    rows["9b_decode_b64"] = {"tok_per_s": B / t, "ms_per_step": t * 1e3}

    xp = torch.randn(prefill_prefix, d9["hidden"], generator=gen).bfloat16().float()

    def prefill():
        lay.prefill(xp, torch.zeros(d9["num_v_heads"], 128, 128), torch.zeros(syn.conv_dim(d9), 3))

    t = _median_time(prefill)
    rows["9b_prefill_16k"] = {"tok_per_s": prefill_prefix / t, "ms_16k_extrapolated": t * 16384 / prefill_prefix * 1e3,
                              "note": f"extrapolated from a {prefill_prefix}-token prefix (time is linear in T)"}
    del lay

    d8 = syn.SHAPES["0.8b"]
    w8, g8 = syn.make_weights(d8, seed=0)
    lay8 = GDNLayerTorchCPU(w8, d8)
    x8, s8 = syn.make_inputs(d8, 1, 1, g8, state_std=0.01)
    conv8 = torch.zeros(1, syn.conv_dim(d8), 3)
    t = _median_time(lambda: lay8.decode(x8[:, 0], s8, conv8))
    rows["0.8b_decode_b1"] = {"tok_per_s": 1 / t, "us_per_step": t * 1e6}

    # side figure: the fp64 C oracle (naive loops, OpenMP) on the headline workload
    oracle.set_threads(threads)
    dm = oracle.dims(d9["hidden"], d9["num_k_heads"], d9["num_v_heads"], 128, 128)
    wn = {k: v.float().numpy() for k, v in w9.items()}
    rec_o = rec.numpy().copy()
    conv_o = np.zeros((B, syn.conv_dim(d9), 3), np.float32)
    xo = x.numpy()[:, None]
    oracle.layer_forward(dm, wn, xo, rec_o, conv_o)
    n, t0 = 0, time.perf_counter()
    while n < 1 or time.perf_counter() - t0 < oracle_seconds:
        oracle.layer_forward(dm, wn, xo, rec_o, conv_o)
        n += 1
    rows["9b_decode_b64_fp64_oracle"] = {"tok_per_s": B * n / (time.perf_counter() - t0),
                                         "note": "fp64 naive-loop oracle, side figure only"}
    head = rows["9b_decode_b64"]
    return {"value": head["tok_per_s"], "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "fp32 torch restatement of the reference's CPU path (oracle/torch_ref.py), 9B decode at "
                      "batch 64: median of 20 steps after 10 warm-ups",
            "cpu_model": _cpu_model(), "rows": rows, "seconds": time.perf_counter() - t_start}


CAL_BYTES = 1 << 30      # the calibration copy in the counter passes


def pmc_child(steps=4):
    """Workload of one counter pass: a 1 GiB device copy (calibrates the counter against bytes that are
    known to move), then `steps` decode steps of one 9B-shape layer at batch 64."""
    import torch

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
    from linear_attention_op_amd import synthetic as syn

    dev = torch.device("cuda", 0)
    src = torch.ones(CAL_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    d = syn.SHAPES["9b"]
    w, _ = syn.make_weights(d, seed=2)
    lay = Qwen35GatedDeltaNetHIP(w, dims=d, batch=64, max_tokens=64, out_dtype=LAYER_OUT)
    lay.set_state(rec=torch.randn(64, d["num_v_heads"], 128, 128, device=dev) * 0.01)
    x = torch.randn(64, 1, d["hidden"], device=dev).to(torch.bfloat16)
    for _ in range(steps):
        lay(x)
    torch.cuda.synchronize()
    lay.close()


def profile_child(which):
    """Workload for an external profiler (rocprofv3 --kernel-trace / --pmc put this process after `--`):
    `decode`: 9B decode at batch 64, 4 layer copies rotated as in the benchmark, SETTLE_S seconds of steps then
    16 more;
    `prefill`: one 16384-token prefill of a 9B layer, SETTLE_S seconds of prefills then 4 more;
    `small`: 9B decode at batch 1 and at batch 8, then the 0.8B shape at batch 1, 8 layer copies each rotated,
    SETTLE_S seconds of steps then 16 more each.
    A kernel trace of these averages over every call: almost all of them run at settled clocks."""
    import torch

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
    from linear_attention_op_amd import synthetic as syn

    dev = torch.device("cuda", 0)
    d = syn.SHAPES["9b"]
    w, _ = syn.make_weights(d, seed=2)
    if which == "small":
        for shape, B in (("9b", 1), ("9b", 8), ("0.8b", 1)):
            ds = syn.SHAPES[shape]
            ws, _ = syn.make_weights(ds, seed=0)
            layers = []
            for i in range(8):
                gg = torch.Generator(device=dev).manual_seed(200 + i)
                wi = {k: (torch.randn(v.shape, generator=gg, device=dev) * v.float().std()).to(v.dtype)
                      if k.startswith("w_") or k == "conv_w" else v for k, v in ws.items()}
                lay = Qwen35GatedDeltaNetHIP(wi, dims=ds, batch=B, max_tokens=64, out_dtype=LAYER_OUT)
                lay.set_state(rec=torch.randn(B, ds["num_v_heads"], 128, 128, device=dev) * 0.01)
                layers.append(lay)
            x = torch.randn(B, 1, ds["hidden"], device=dev).to(torch.bfloat16)
            it = iter(range(1 << 62))
            settle(lambda: layers[next(it) % 8](x))
            for i in range(16):
                layers[i % 8](x)
            torch.cuda.synchronize()
            for lay in layers:
                lay.close()
    elif which == "decode":
        layers = []
        for i in range(4):
            gg = torch.Generator(device=dev).manual_seed(100 + i)
            wi = w if i == 0 else {k: (torch.randn(v.shape, generator=gg, device=dev) * v.float().std()).to(v.dtype)
                                   if k.startswith("w_") or k == "conv_w" else v for k, v in w.items()}
            lay = Qwen35GatedDeltaNetHIP(wi, dims=d, batch=64, max_tokens=64, out_dtype=LAYER_OUT)
            lay.set_state(rec=torch.randn(64, d["num_v_heads"], 128, 128, device=dev) * 0.01)
            layers.append(lay)
        x = torch.randn(64, 1, d["hidden"], device=dev).to(torch.bfloat16)
        it = iter(range(1 << 62))
        settle(lambda: layers[next(it) % 4](x))
        for i in range(16):
            layers[i % 4](x)
    else:
        lay = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=16384, out_dtype=LAYER_OUT)
        x = torch.randn(1, 16384, d["hidden"], device=dev).to(torch.bfloat16)

        def once():
            lay.reset_state()
            lay(x)

        settle(once)
        for _ in range(4):
            once()
    torch.cuda.synchronize()
    print(f"profile child {which}: done", flush=True)


def measure_traffic(kernel="mixer_kernel", timeout=180):
    """HBM bytes per launch of `kernel` from two rocprofv3 counter passes over `pmc_child` (FETCH_SIZE,
    then WRITE_SIZE, KiB per dispatch), each scaled by what the same counter reads for the 1 GiB copy.
    Runs before this process touches the GPU.  Returns (traffic dict, None) or (None, reason)."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        tmp = tempfile.mkdtemp(prefix="gdn_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", tmp, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--pmc-child"]
        env = dict(os.environ, TMPDIR="/tmp")
        print(f"[bench] counter pass {counter}", file=sys.stderr, flush=True)
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout, stdout=subprocess.DEVNULL,
                               stderr=subprocess.PIPE, text=True)
        except subprocess.TimeoutExpired:
            return None, f"{counter} pass timed out"
        rows = []
        for root, _, files in os.walk(tmp):
            for f in files:
                if f.endswith("counter_collection.csv"):
                    with open(os.path.join(root, f)) as fh:
                        rows += list(csv.DictReader(fh))
        shutil.rmtree(tmp, ignore_errors=True)
        if not rows:
            return None, f"{counter} pass wrote no counters (rc {r.returncode}): {r.stderr[-300:]}"
        cal = max((float(x["Counter_Value"]) for x in rows if "copyBuffer" in x["Kernel_Name"]), default=0.0)
        vals = [float(x["Counter_Value"]) for x in rows if kernel in x["Kernel_Name"]]
        if cal <= 0 or not vals:
            return None, f"{counter} pass: no calibration copy or no {kernel} dispatch"
        scale = CAL_BYTES / (cal * 1024)        # bytes per counted KiB
        out[counter] = {"kib_per_dispatch": sum(vals) / len(vals), "scale": scale, "dispatches": len(vals),
                        "bytes": sum(vals) / len(vals) * 1024 * scale}
    return {"bytes": out["FETCH_SIZE"]["bytes"] + out["WRITE_SIZE"]["bytes"], "passes": out}, None


STREAM_MODES = {0: "read", 1: "write", 2: "copy", 3: "in_place"}


def hbm_ceiling(buf_bytes=512 << 20, copies=4, reps=4, sweep_log=None):
    """The HBM rate a purpose-built stream kernel reaches on this device (csrc/hbm_stream.hip): read-only,
    write-only, copy and in-place read + write, each over `copies` rotating buffers of `buf_bytes` (more than
    the 256 MB Infinity Cache in all), swept over 16-byte accesses in flight per thread (1-16), non-temporal
    accesses off / on and the grid size.  Returns {mode: best row} (GB/s, the fraction of 8 TB/s and the
    configuration); every row goes to `sweep_log` if given."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "linear_attention_op_amd", "libgdn_stream.so"))
    fn = lib.gdn_stream_run
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    src = [torch.ones(buf_bytes // 4, device="cuda") for _ in range(copies)]
    dst = [torch.zeros(buf_bytes // 4, device="cuda") for _ in range(copies)]
    sink = torch.zeros(256, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    n4 = buf_bytes // 16
    best = {}
    rows = []
    for mode in (0, 1, 2, 3):
        moved = buf_bytes * (2 if mode in (2, 3) else 1)
        for unroll in (1, 2, 4, 8, 16):
            for nt in (0, 1):
                for blocks in (1024, 2048, 4096, 8192, -1):
                    nb = blocks if blocks > 0 else (n4 + 256 * unroll - 1) // (256 * unroll)

                    def run(i):
                        rc = fn(mode, unroll, nt, ctypes.c_void_p(src[i].data_ptr()),
                                ctypes.c_void_p(dst[i].data_ptr()), buf_bytes, nb, ctypes.c_void_p(sink.data_ptr()), st)
                        if rc:
                            raise RuntimeError(f"gdn_stream_run returned {rc}")

                    for i in range(copies):
                        run(i)
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for r in range(reps * copies):
                        run(r % copies)
                    e1.record()
                    torch.cuda.synchronize()
                    sec = e0.elapsed_time(e1) / 1e3 / (reps * copies)
                    row = {"mode": STREAM_MODES[mode], "unroll": unroll, "nontemporal": nt, "blocks": nb,
                           "GBps": moved / sec / 1e9, "frac": moved / sec / HBM_PEAK}
                    rows.append(row)
                    if sweep_log:
                        print(json.dumps(row), file=sweep_log, flush=True)
                    if row["GBps"] > best.get(row["mode"], {"GBps": 0})["GBps"]:
                        best[row["mode"]] = row
    del src, dst
    torch.cuda.synchronize()
    return best


def prefill_bench(w, d, T, steps, weight_dtype="bf16"):
    """One sequence of T tokens through one layer from a zero state (in_proj GEMM, chunked mixer, out_proj
    GEMM), `steps` times: the HIP-event layer time per prefill and its bf16-MFMA roofline fraction (E4M3 and
    MXFP4 weights are widened to bf16 on the way into LDS, so the MFMA work is the same)."""
    import torch

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP

    dev = torch.device("cuda", 0)
    lay = Qwen35GatedDeltaNetHIP(w, dims=d, batch=1, max_tokens=T, weight_dtype=weight_dtype, out_dtype=LAYER_OUT)
    x = torch.randn(1, T, d["hidden"], device=dev).to(torch.bfloat16)

    def once():
        lay.reset_state()
        lay(x)

    settle(once)
    torch.cuda.synchronize()
    lay.profile(steps)
    t0 = time.perf_counter()
    for _ in range(steps):
        lay.reset_state()
        lay(x)
    torch.cuda.synchronize()
    pe = (time.perf_counter() - t0) / steps
    ms, n = lay.profile_read()
    ev = ms["total"] / max(n, 1) / 1e3
    flops = prefill_flops_per_token(d) * T
    out = {"tokens": T, "weights": weight_dtype, "tok_per_s": T / ev, "ms": ev * 1e3, "wall_ms": pe * 1e3,
           "stage_ms": {k: v / max(n, 1) for k, v in ms.items()},
           "roofline": {"bound": "mfma", "achieved": flops / ev / 1e12, "peak": BF16_PEAK / 1e12,
                        "unit": "TFLOP/s", "frac": flops / ev / BF16_PEAK, "flops": flops}}
    print(f"[bench] prefill T={T} {weight_dtype}: {ev * 1e3:.2f} ms, {T / ev:.0f} tok/s, stages (ms) "
          f"{ {k: round(v / max(n, 1), 3) for k, v in ms.items()} }", file=sys.stderr, flush=True)
    lay.close()
    return out


def small_batch_decode(shape, B, copies=8, steps=400, warmup=40, weight_dtype="bf16"):
    """Decode latency of one layer at a small batch, one HIP graph per layer copy (launch overhead is most
    of such a step), rotating over `copies` layers so that the weights come from HBM."""
    import torch

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
    from linear_attention_op_amd import synthetic as syn

    d = syn.SHAPES[shape]
    dev = torch.device("cuda", 0)
    w0, _ = syn.make_weights(d, seed=0)
    layers, xin = [], []
    for i in range(copies):
        gg = torch.Generator(device=dev).manual_seed(200 + i)
        w = {k: (torch.randn(v.shape, generator=gg, device=dev) * v.float().std()).to(v.dtype)
             if k.startswith("w_") or k == "conv_w" else v for k, v in w0.items()}
        lay = Qwen35GatedDeltaNetHIP(w, dims=d, batch=B, max_tokens=64, weight_dtype=weight_dtype, out_dtype=LAYER_OUT)
        lay.set_state(rec=torch.randn(B, d["num_v_heads"], d["head_k_dim"], d["head_v_dim"], device=dev) * 0.01)
        layers.append(lay)
        xin.append(torch.randn(B, 1, d["hidden"], device=dev).to(torch.bfloat16))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for lay, x in zip(layers, xin):
            lay(x)
    torch.cuda.current_stream().wait_stream(side)
    graphs = []
    for lay, x in zip(layers, xin):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            lay(x)
        graphs.append(g)
    it = iter(range(1 << 62))
    settle(lambda: graphs[next(it) % copies].replay())
    for i in range(warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / steps * 1e6
    W, s = decode_bytes(d, B, weight_dtype)
    out = {"shape": shape, "batch": B, "weights": weight_dtype, "us_per_step": us, "tok_per_s": B / (us * 1e-6),
           "hbm_frac": (W + B * s) / (us * 1e-6) / HBM_PEAK, "mode": "HIP graph per step"}
    for lay in layers:
        lay.close()
    return out


def stack_bench(d, n_layers=24, n_prefill=8, prefill_len=2048, n_decode=56, steps=3, warmup=1, seed=4):
    """Continuous batching through a stack of 9B-shape layers with the decoder RMSNorm between layers
    (synthetic.continuous_batch, seed 4): every step carries the next prefill_len tokens of n_prefill prompts
    (chunked prefill, states carried) and one token for each of n_decode streams, in one variable-length
    launch per layer.  The decode streams start from 0.01 randn states (a GDN state has constant size, so a
    long context only changes its values)."""
    import torch

    from linear_attention_op_amd import Qwen35GDNStackHIP
    from linear_attention_op_amd import synthetic as syn

    layers, cu, x, s0 = syn.continuous_batch(d, n_layers=n_layers, n_prefill=n_prefill, prefill_len=prefill_len,
                                             n_decode=n_decode, seed=seed)
    n_seq, rows = n_prefill + n_decode, cu[-1]
    stack = Qwen35GDNStackHIP(layers, dims=d, batch=n_seq, max_slots=n_seq, max_tokens=rows,
                              inter_norm=True, out_dtype=LAYER_OUT)
    del layers
    slots = torch.arange(n_seq, dtype=torch.int32, device="cuda")
    for L, s in zip(stack.layers, s0):
        L.set_state(rec=s, slot_ids=slots[n_prefill:])
    del s0
    xs = [x, torch.roll(x, 1, 0)]
    it = iter(range(1 << 62))
    settle(lambda: stack.forward_varlen(xs[next(it) % 2], cu, slots))
    for i in range(warmup):
        stack.forward_varlen(xs[i % 2], cu, slots)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        stack.forward_varlen(xs[i % 2], cu, slots)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    stack.close()
    flops = n_layers * rows * prefill_flops_per_token(d)
    return {"workload": f"{n_layers} 9B-shape GDN layers with RMSNorm between layers, continuous batch of "
                        f"{n_prefill} prefills x {prefill_len} tokens + {n_decode} decode streams per step",
            "tokens_per_step": rows, "ms_per_step": dt * 1e3, "tok_per_s": rows / dt, "steps": steps,
            "roofline": {"bound": "mfma", "achieved": flops / dt / 1e12, "peak": BF16_PEAK / 1e12,
                         "unit": "TFLOP/s", "frac": flops / dt / BF16_PEAK, "flops": flops}}


def main():
    if "--pmc-child" in sys.argv:
        pmc_child()
        return
    if "--profile-child" in sys.argv:
        profile_child(sys.argv[sys.argv.index("--profile-child") + 1])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--copies", type=int, default=4, help="independent layers rotated through (defeats MALL)")
    ap.add_argument("--prefill-len", type=int, default=16384)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--graph", type=int, default=0,
                    help="1: replay the decode step from HIP graphs; 0: launch eagerly (faster here: 104 vs 112 us)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fp8", action="store_true", help="skip the FP8- and MXFP4-weight decode and prefill measurements")
    ap.add_argument("--no-small", action="store_true", help="skip the batch-1/8 decode latencies")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the 24-layer continuous-batching stack (8 x 2048 prefill + 56 decode per step)")
    ap.add_argument("--stream-log", default=None, help="write every row of the HBM stream sweep to this file")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes (required when bench.py itself runs under rocprofv3)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the layer shards by v-head "
              "or by sequence across GPUs only in design); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    traffic, traffic_note = (None, "skipped (--no-traffic)") if args.no_traffic else measure_traffic()
    if traffic_note:
        print(f"[bench] traffic: {traffic_note}", file=sys.stderr, flush=True)

    import torch

    from linear_attention_op_amd import Qwen35GatedDeltaNetHIP
    from linear_attention_op_amd import synthetic as syn

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    d = syn.SHAPES["9b"]
    B, L = args.batch, args.copies
    print(f"[bench] building {L} 9B-shape layers, batch {B}", file=sys.stderr, flush=True)

    w0, gen = syn.make_weights(d, seed=2)

    def copy_weights(i):
        if i == 0:
            return w0
        # further copies: same distribution, drawn on the GPU (values do not affect timing)
        gg = torch.Generator(device=dev).manual_seed(100 + i)
        return {k: (torch.randn(v.shape, generator=gg, device=dev) * v.float().std()).to(v.dtype)
                if k.startswith("w_") or k == "conv_w" else v for k, v in w0.items()}

    layers = []
    for i in range(L):
        lay = Qwen35GatedDeltaNetHIP(copy_weights(i), dims=d, batch=B, max_tokens=max(B, 64), out_dtype=LAYER_OUT)
        s0 = torch.randn(B, d["num_v_heads"], 128, 128, device=dev) * 0.01
        lay.set_state(rec=s0)
        layers.append(lay)
    xs = [(torch.randn(B, 1, d["hidden"], device=dev)).to(torch.bfloat16) for _ in range(4)]
    torch.cuda.synchronize()

    # eager warm-up, then one HIP graph per layer copy for the decode step (the counterpart of the
    # reference's traced decode, wormhole_n150/qwen3.5_0.8B/bench_decode.py:44-60)
    it = iter(range(1 << 62))
    settle(lambda: (lambda i: layers[i % L](xs[i % 4]))(next(it)))
    for i in range(args.warmup):
        layers[i % L](xs[i % 4])
    torch.cuda.synchronize()
    steps_fn = []
    if args.graph:
        xin = [xs[i % 4].clone() for i in range(L)]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(L):
                layers[i](xin[i])
        torch.cuda.current_stream().wait_stream(side)
        graphs = []
        for i in range(L):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                layers[i](xin[i])
            graphs.append(g)
        for i in range(args.warmup):
            graphs[i % L].replay()
        steps_fn = [g.replay for g in graphs]
    else:
        steps_fn = [(lambda i=i: layers[i](xs[i % 4])) for i in range(L)]
    torch.cuda.synchronize()

    # timed region: exactly `steps` decode steps, synchronised on both sides
    t0 = time.perf_counter()
    for i in range(args.steps):
        steps_fn[i % L]()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # stage breakdown: the same steps run eagerly with HIP events recorded on the launch stream at the
    # stage boundaries (in_proj | mixer | out_proj)
    for lay in layers:
        lay.profile(args.steps)
    torch.cuda.synchronize()
    for i in range(args.steps):
        layers[i % L](xs[i % 4])
    torch.cuda.synchronize()
    stage = {"in_proj": 0.0, "mixer": 0.0, "out_proj": 0.0, "total": 0.0}
    calls = 0
    for lay in layers:
        ms, n = lay.profile_read()
        calls += n
        for k in stage:
            stage[k] += ms[k]
        lay.profile(0)
    stage_avg_ms = {k: v / max(calls, 1) for k, v in stage.items()}

    ms_per_step = elapsed * 1e3 / args.steps
    value = B / (ms_per_step / 1e3)
    W, s = decode_bytes(d, B)
    step_bytes = W + B * s
    mix_bytes = B * mixer_bytes_per_seq(d)
    mix_s = stage_avg_ms["mixer"] / 1e3
    roofline = {"bound": "hbm", "achieved": mix_bytes / mix_s / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": mix_bytes / mix_s / HBM_PEAK, "traffic": traffic["bytes"] if traffic else None,
                "kernel": "mixer_kernel<128,128>", "bytes_per_launch": mix_bytes,
                "avg_launch_us": stage_avg_ms["mixer"] * 1e3,
                "traffic_detail": traffic["passes"] if traffic else traffic_note}
    layer_roof = {"bytes_per_step": step_bytes, "achieved_GBps": step_bytes / (ms_per_step / 1e3) / 1e9,
                  "frac": step_bytes / (ms_per_step / 1e3) / HBM_PEAK,
                  "event_step_us": stage_avg_ms["total"] * 1e3,
                  "event_frac": step_bytes / (stage_avg_ms["total"] / 1e3) / HBM_PEAK,
                  "stage_us": {k: v * 1e3 for k, v in stage_avg_ms.items()}}
    # the practical ceiling for the mixer's traffic: the best in-place read + write stream (the state's access
    # pattern) a purpose-built kernel reaches here, and the best read-only, write-only and copy streams
    ceiling = hbm_ceiling(sweep_log=open(args.stream_log, "w") if args.stream_log else None)
    roofline["frac_of_stream"] = roofline["achieved"] / ceiling["in_place"]["GBps"]
    print(f"[bench] stream ceiling: " + ", ".join(f"{k} {v['GBps']:.0f} GB/s ({v['frac'] * 100:.0f}%)"
                                                   for k, v in ceiling.items()) +
          f"; mixer {roofline['achieved']:.0f} GB/s", file=sys.stderr, flush=True)
    print(f"[bench] decode B={B}: {ms_per_step * 1e3:.1f} us/step wall ({'graph' if args.graph else 'eager'}), "
          f"eager stages (us) "
          f"{ {k: round(v * 1e3, 1) for k, v in stage_avg_ms.items()} }", file=sys.stderr, flush=True)
    for lay in layers[1:]:
        lay.close()
    del layers[1:]

    # the same decode step on low-precision weights: E4M3 (one byte per weight, per-row scales), MXFP4 (half a
    # byte, a scale per 32) and MXINT8 (one byte, a scale per 32: the bfloat8_b counterpart)
    lowp = {}
    if not args.no_fp8:
        for wd, desc in (("fp8", "E4M3, one fp32 scale per row (a|b rows bf16)"),
                         ("mxfp4", "MXFP4 (E2M1, one E8M0 scale per 32; a|b rows bf16)"),
                         ("mxint8", "MXINT8 (int8 codes, one E8M0 scale per 32; a|b rows bf16)")):
            print(f"[bench] {wd}-weight decode, {L} copies", file=sys.stderr, flush=True)
            lays = []
            for i in range(L):
                lay = Qwen35GatedDeltaNetHIP(copy_weights(i), dims=d, batch=B, max_tokens=max(B, 64),
                                             weight_dtype=wd, out_dtype=LAYER_OUT)
                lay.set_state(rec=torch.randn(B, d["num_v_heads"], 128, 128, device=dev) * 0.01)
                lays.append(lay)
            wall, st = eager_decode(lays, xs, args.steps, args.warmup)
            Wq, sq = decode_bytes(d, B, wd)
            bq = Wq + B * sq
            lowp[wd] = {"ms_per_step": wall, "tok_per_s": B / (wall / 1e3), "bytes_per_step": bq,
                        "frac": bq / (wall / 1e3) / HBM_PEAK, "event_step_us": st["total"] * 1e3,
                        "stage_us": {k: v * 1e3 for k, v in st.items()}, "weights": desc}
            print(f"[bench] {wd} decode B={B}: {wall * 1e3:.1f} us/step wall, stages (us) "
                  f"{ {k: round(v * 1e3, 1) for k, v in st.items()} }", file=sys.stderr, flush=True)
            for lay in lays:
                lay.close()
            del lays
        # in_proj weight stream (q|k|v|z codes + scales + bf16 a|b rows) over the in_proj stage time
        H, nv = d["hidden"], d["num_v_heads"]
        n1 = 2 * d["num_k_heads"] * 128 + 2 * nv * 128
        lowp["fp8"]["in_proj_GBps"] = (n1 * H + 4 * n1 + 2 * 2 * nv * H) / (lowp["fp8"]["stage_us"]["in_proj"] / 1e6) / 1e9

    prefill = None
    prefill_lowp = None
    prefill_4k = None
    if not args.no_prefill:
        prefill = prefill_bench(w0, d, args.prefill_len, args.prefill_steps)
        # the other prefill length of the 9B prefill configuration (one sequence of 4096 tokens)
        prefill_4k = prefill_bench(w0, d, 4096, 2 * args.prefill_steps)
        if not args.no_fp8:
            prefill_lowp = [prefill_bench(w0, d, args.prefill_len, args.prefill_steps, wd)
                            for wd in ("fp8", "mxfp4", "mxint8")]

    # small-batch decode latency (the reference's headline configurations are batch 1)
    small = None
    if not args.no_small:
        small = [small_batch_decode("0.8b", 1), small_batch_decode("9b", 1), small_batch_decode("9b", 8)]
        if not args.no_fp8:
            small += [small_batch_decode("9b", 1, weight_dtype=wd) for wd in ("fp8", "mxfp4", "mxint8")]
        for r in small:
            print(f"[bench] decode {r['shape']} B={r['batch']} {r['weights']}: {r['us_per_step']:.1f} us/step (graph), "
                  f"{r['hbm_frac'] * 100:.0f}% of HBM roofline", file=sys.stderr, flush=True)

    stack = None
    if not args.no_stack:
        print("[bench] 24-layer continuous-batching stack", file=sys.stderr, flush=True)
        stack = stack_bench(d)
        print(f"[bench] stack: {stack['ms_per_step']:.1f} ms/step, {stack['tok_per_s']:.0f} tok/s", file=sys.stderr,
              flush=True)

    cpu = None
    if not args.no_cpu:
        print("[bench] timing the reference's CPU path (fp32 torch restatement) on the host", file=sys.stderr,
              flush=True)
        cpu = cpu_baseline({k: v.float().cpu() for k, v in w0.items()})
        print(f"[bench] CPU baseline ({cpu['cores']} threads, {cpu['cpu_model']}): "
              f"{ {k: round(v['tok_per_s'], 1) for k, v in cpu['rows'].items()} } tok/s", file=sys.stderr,
              flush=True)

    line = {
        "metric": METRIC, "value": value, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"9B-shape GDN layer decode, batch {B}, one token per sequence per step, "
                               f"rotating over {L} layer copies" + (", HIP-graph replay" if args.graph else ""),
                   "hidden": d["hidden"], "num_k_heads": d["num_k_heads"], "num_v_heads": d["num_v_heads"],
                   "head_dim": 128, "batch": B, "state_dtype": "fp32", "weights": "bf16 N(0,0.02) seed 2"},
        "roofline": roofline, "layer_roofline": layer_roof, "stream_ceiling": ceiling, "prefill": prefill,
        "prefill_t4096": prefill_4k,
        "prefill_lowp_weights": prefill_lowp, "stack": stack, "fp8_decode": lowp.get("fp8"),
        "mxfp4_decode": lowp.get("mxfp4"), "mxint8_decode": lowp.get("mxint8"),
        "small_batch_decode": small,
        "cpu_baseline": cpu,
        "settle": {"seconds": SETTLE_S, "what": "untimed runs of each measured workload before its warm-up steps, "
                                                "so that the clocks have left their idle state"},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
