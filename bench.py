#!/usr/bin/env python3
"""Benchmark: causal attention fwd+bwd on one MI355X (BASELINE.json metric).

Workload (one "step"): forward + backward of causal scaled-dot-product attention,
B=8 H=12 T=1024 d=64, fp32 (configs[1] is its forward half).  Q, K, V,
dO are synthetic N(0, 1) tensors already resident in HBM; outputs, LSE and the backward
workspace are preallocated, so the timed region is kernels only.

Prints ONE JSON line.  `value` is TFLOP/s by the FA2 convention: the forward is two
matmuls of 2*T^2*d flops per (b, h), causal counts half of T^2, so fwd = 2*B*H*T^2*d =
12.885 GFLOP; the backward is 2.5x that; fwd+bwd = 3.5x -> 45.097 GFLOP per step.

  python bench.py [--gpus 1] [--steps 100] [--warmup 50] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys

# Workloads.  The default, c3, is the headline metric; c4 is the
# bf16 long-context config, c5 the NanoGPT training step, and "layer" the reference test's
# whole attention layer, each reported separately (python bench.py --workload c4).
WORKLOADS = {
    "c3": dict(B=8, H=12, T=1024, D=64, dtype="f32", std=1.0, peak=157.3,
               metric="causal attn fwd+bwd TFLOP/s + % MFMA peak, B8 H12 T1024 d64 fp32, 1 GPU",
               label="causal SDPA fwd+bwd, B8 H12 T1024 d64 fp32 (BASELINE configs[2])"),
    "c5": dict(B=16, H=6, T=256, D=64, dtype="f32", std=1.0, peak=157.3,
               metric="NanoGPT config-5 training step tokens/s (attention on ctattn), fp32, 1 GPU",
               label="NanoGPT 6L d384 6H T256 B16 vocab65 GELU, Adam lr 3e-4, fp32 (BASELINE configs[4])"),
    "c5n": dict(B=16, H=6, T=256, D=64, dtype="f32", std=1.0, peak=157.3,
                metric="NanoGPT config-5 training step tokens/s (native host, every layer on libctattn), "
                       "fp32, 1 GPU",
                label="NanoGPT 6L d384 6H T256 B16 vocab65 GELU causal, Adam lr 3e-4, fp32 (BASELINE "
                      "configs[4]) on the native C++ host: forward, loss, backward, Adam"),
    "layer": dict(B=8, H=16, T=1024, D=64, E=1024, dtype="f32", std=1.0, peak=157.3,
                  metric="attention layer (QKV proj + attention + out proj) fwd+bwd TFLOP/s, "
                         "B8 N1024 E1024 H16 D64 fp32, 1 GPU",
                  label="AttentionFloat(input_dim=1024, num_heads=16, head_dim=64) on X[8, 1024, 1024], "
                        "non-causal, the reference test's configuration (test_flash_attention.py:9-12) at N=1024"),
    "layerbf": dict(B=8, H=16, T=1024, D=64, E=1024, dtype="bf16", std=1.0, peak=2516.6,
                    metric="attention layer (QKV proj + attention + out proj) fwd+bwd TFLOP/s, "
                           "B8 N1024 E1024 H16 D64 bf16, 1 GPU",
                    label="AttentionBFloat(input_dim=1024, num_heads=16, head_dim=64) on X[8, 1024, 1024], "
                          "non-causal: the reference test's configuration in bf16 storage (fp32 accumulation; "
                          "projections on the 16-bit MFMA GEMMs)"),
    "c4": dict(B=1, H=32, T=8192, D=128, dtype="bf16", std=0.5, peak=2516.6,
               metric="causal attn fwd+bwd TFLOP/s + % MFMA peak, B1 H32 T8192 d128 bf16, 1 GPU",
               label="causal SDPA fwd+bwd, B1 H32 T8192 d128 bf16 in / fp32 accumulate (BASELINE configs[3])"),
    "c4h": dict(B=1, H=32, T=8192, D=128, dtype="f16", std=0.5, peak=2516.6,
                metric="causal attn fwd+bwd TFLOP/s + % MFMA peak, B1 H32 T8192 d128 fp16, 1 GPU",
                label="causal SDPA fwd+bwd, B1 H32 T8192 d128 fp16 in / fp32 accumulate (BASELINE configs[3] "
                      "shape in the reference's Half precision)"),
    "tensor": dict(B=1, H=1, T=1, D=1, dtype="f32", std=1.0, peak=8000.0,
                   metric="Tensor operations HBM GB/s (elementwise add of 2 x 256 MiB fp32), 1 GPU",
                   label="FloatTensor a + b on 64 Mi elements (768 MiB moved), with sum(), bfloat() cast, "
                         "transpose(1, 0) of 8192 x 8192 and a 4096^3 matmul alongside"),
    "c3d": dict(B=8, H=12, T=1024, D=64, dtype="f64", std=1.0, peak=78.6,
                metric="causal attn fwd+bwd TFLOP/s, B8 H12 T1024 d64 fp64, 1 GPU",
                label="causal SDPA fwd+bwd, B8 H12 T1024 d64 fp64 (the headline shape in the reference's "
                      "Double precision; fp64 MFMA kernels)"),
}
TORCH_DTYPE = {"f32": "float32", "bf16": "bfloat16", "f16": "float16", "f64": "float64"}
B, H, T, D = 8, 12, 1024, 64
CAUSAL = True
FWD_FLOP = 4.0 * B * H * T * T * D / 2.0  # QK^T + PV, 2*T^2*d each; causal = half of T^2
BWD_FLOP = 2.5 * FWD_FLOP
STEP_FLOP = FWD_FLOP + BWD_FLOP
PEAK_F32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
METRIC = WORKLOADS["c3"]["metric"]
HERE = os.path.dirname(os.path.abspath(__file__))
# rocprofv3 counter summaries of the attention kernels at a workload's shape (bench.* lines)
COUNTERS_FILES = {
    "c3": os.path.join(HERE, "profiles", "attn_f32_c3_counters.txt"),
    "c4": os.path.join(HERE, "profiles", "attn_bf16_c4_counters.txt"),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def read_profile_figures(path):
    """Machine-readable figures of a committed rocprofv3 summary: every line of the form
    ``bench.<key>: <number>``.  Empty if the file is absent."""
    figs = {}
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("bench.") and ":" in line:
                    key, val = line[len("bench."):].split(":", 1)
                    figs[key.strip()] = float(val)
    except OSError:
        pass
    return figs


def cpu_baseline(seconds: float):
    """The north star's CPU comparator: torch.nn.functional.scaled_dot_product_attention in
    fp32 on CPU tensors, forward + backward of the full headline step on every host thread
    (the routine the reference's test_flash_attention.py:49 checks against), median of
    repetitions over about `seconds`.  Beside it, the C restatement of the reference
    algorithm (oracle/attn_online.c: fp64 tiled online softmax, recompute backward; scalar,
    one thread) over one (b, h) slice after another until `seconds` have elapsed."""
    sys.path.insert(0, HERE)
    import time

    import numpy as np

    from oracle import c_oracle, torch_cpu

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    med, reps, threads = torch_cpu.time_fwd_bwd((B, H, T, D), CAUSAL, seconds=seconds,
                                               threads=threads)
    rng = np.random.default_rng(3)
    try:
        c_oracle.load()
    except FileNotFoundError:  # the checker is built by build(); build it here if absent
        import subprocess
        subprocess.run(["make", "-C", os.path.join(HERE, "oracle")], check=True)
        c_oracle.load()
    busy, done = 0.0, 0
    while done < B * H and (done == 0 or busy < seconds):
        q, k, v, do = (rng.standard_normal((1, 1, T, D)) for _ in range(4))
        t0 = time.perf_counter()
        o, lse = c_oracle.fwd(q, k, v, CAUSAL)
        c_oracle.bwd(q, k, v, o, do, lse, CAUSAL)
        busy += time.perf_counter() - t0
        done += 1
    return {
        "value": STEP_FLOP / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        # torch's CPU SDPA (a library routine, the reference test's comparator), not a port of
        # the reference: the C port's figure is c_port_value beside it.
        "kind": "torch-cpu",
        "sample": (f"oracle/torch_cpu.py: torch.nn.functional.scaled_dot_product_attention fp32 "
                   f"causal fwd+bwd on CPU tensors (the comparator of the reference's "
                   f"test_flash_attention.py:49), the full B{B} H{H} T{T} d{D} step on {threads} "
                   f"host threads, median of {reps} reps = {med * 1e3:.1f} ms/step"),
        "c_port_value": STEP_FLOP * done / (B * H) / busy / 1e12,
        "c_port_sample": (f"oracle/attn_online.c (fp64, scalar, 1 thread) fwd+bwd of {done} of the "
                          f"{B * H} (b, h) slices in {busy:.1f} s ({busy / done * B * H:.1f} s per "
                          f"full step)"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    # After the --warmup steps, more untimed steps run until this much wall time has passed:
    # the GPU clocks take a few hundred ms of load to settle, and with a handful of warm-up
    # steps the first timed steps run about 7-10% slower.  Reported as config.preroll_*.
    ap.add_argument("--preroll-ms", type=float, default=1000.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c3")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (rocprofv3 --pmc calibration of "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count)")
    args = ap.parse_args()

    global B, H, T, D, FWD_FLOP, BWD_FLOP, STEP_FLOP, PEAK_F32_MFMA, METRIC
    wl = WORKLOADS[args.workload]
    B, H, T, D = wl["B"], wl["H"], wl["T"], wl["D"]
    FWD_FLOP = 4.0 * B * H * T * T * D / 2.0
    BWD_FLOP = 2.5 * FWD_FLOP
    STEP_FLOP = FWD_FLOP + BWD_FLOP
    PEAK_F32_MFMA = wl["peak"]
    METRIC = wl["metric"]
    if args.workload != "c3":
        args.no_cpu_baseline = True  # the CPU baseline is quoted for the headline config

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this build measures one GPU "
              f"(the attention path shards by (batch, head) with no exchange between GPUs)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    sys.path.insert(0, HERE)
    import cudatransformer_amd as ct

    dev = torch.device("cuda:0")
    if args.workload == "c5":
        return bench_nanogpt(args, wl, dev)
    if args.workload == "c5n":
        return bench_native_nanogpt(args, wl)
    if args.workload in ("layer", "layerbf"):
        return bench_layer(args, wl)
    if args.workload == "tensor":
        return bench_tensor(args, wl)
    if args.copy_calibration:
        n = 64 << 20  # 64 Mi fp32 = 256 MiB read + 256 MiB written per copy
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": True, "bytes_read_per_copy": 4 * n,
                          "bytes_written_per_copy": 4 * n, "copies": max(args.steps, 1)}),
              flush=True)
        return
    g = torch.Generator(device=dev).manual_seed(2)
    tdt = getattr(torch, TORCH_DTYPE[wl["dtype"]])
    q, k, v, do = ((wl["std"] * torch.randn((B, H, T, D), generator=g, device=dev,
                                            dtype=torch.float32)).to(tdt) for _ in range(4))
    o = torch.empty_like(q)
    lse = torch.empty((B, H, T), device=dev, dtype=torch.float64 if tdt == torch.float64 else torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    # The backward gets the workspace of its fastest path (ctattn_bwd_workspace_bytes_max: at
    # bf16 / fp16 d = 128 the dS tiles, 2.2 GB at c4; the same as the default elsewhere).
    ws_bytes = ct.bwd_workspace_bytes(tdt, B, H, T, D, CAUSAL, fastest=True)
    ws_default = ct.bwd_workspace_bytes(tdt, B, H, T, D, CAUSAL)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    stream = torch.cuda.current_stream()

    def fwd():
        ct.flash_attn_fwd(q, k, v, CAUSAL, out=o, lse=lse, stream=stream)

    def bwd():
        ct.flash_attn_bwd(q, k, v, o, do, lse, CAUSAL, dq=dq, dk=dk, dv=dv, workspace=ws,
                          stream=stream)

    def step():
        fwd()
        bwd()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    preroll_steps, preroll_s = preroll(step, args.preroll_ms)

    # Whole-step timing: exactly K steps between two events on the launch stream.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    log(f"step: {ms_per_step:.4f} ms")

    # Per-phase timing (same stream): forward alone, backward alone.
    def time_phase(fn, reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    fwd_ms = time_phase(fwd, args.steps)
    bwd_ms = time_phase(bwd, args.steps)
    log(f"fwd: {fwd_ms:.4f} ms  bwd: {bwd_ms:.4f} ms")
    layer_ms = time_layer_path(q, do, args) if wl["dtype"] == "f32" else None

    value = STEP_FLOP / (ms_per_step * 1e-3) / 1e12
    achieved = BWD_FLOP / (bwd_ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic",
        "pct_of_peak": round(100.0 * value / PEAK_F32_MFMA, 2),
        "config": {
            "workload": wl["label"],
            "B": B, "H": H, "T": T, "d": D, "causal": CAUSAL,
            "step_gflop": round(STEP_FLOP / 1e9, 3),
            "fwd_ms": round(fwd_ms, 5),
            "bwd_ms": round(bwd_ms, 5),
            # The C++ FlashAttentionLayer path (pybind): computeAttention(save_states=True) +
            # computeBackward per step, output / gradient / workspace allocation included,
            # host wall clock around synchronised steps.
            "layer_path_ms": None if layer_ms is None else round(layer_ms, 5),
            "bwd_workspace_bytes": ws_bytes,
            "bwd_workspace_default_bytes": ws_default,
            "preroll_steps": preroll_steps,
            "preroll_s": round(preroll_s, 3),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attention backward (ctattn_bwd: preprocess + main kernel)",
            "achieved": round(achieved, 3),
            "peak": PEAK_F32_MFMA,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F32_MFMA, 4),
            "traffic": None,
        },
        "cpu_baseline": None,
    }
    if args.workload in COUNTERS_FILES:
        # Counter-derived figures of the same kernels at the same shape, from the committed
        # rocprofv3 --pmc summary: HBM bytes per call (FETCH_SIZE + WRITE_SIZE,
        # copy-calibrated) -> GB/s over this run's measured times, and MFMA utilisation
        # (SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs' active cycles).
        path = COUNTERS_FILES[args.workload]
        figs = read_profile_figures(path)
        if "bwd_traffic_bytes" in figs:
            out["roofline"]["traffic"] = figs["bwd_traffic_bytes"]
            out["roofline"]["hbm_gbs"] = round(figs["bwd_traffic_bytes"] / (bwd_ms * 1e-3) / 1e9, 1)
        for key in ("bwd_mfma_util_pct", "fwd_mfma_util_pct"):
            if key in figs:
                out["roofline"][key] = figs[key]
                out["config"][key] = figs[key]
        if "fwd_traffic_bytes" in figs:
            out["config"]["fwd_hbm_gbs"] = round(figs["fwd_traffic_bytes"] / (fwd_ms * 1e-3) / 1e9, 1)
        if "hbm_gbs" in out["roofline"]:
            out["config"]["bwd_hbm_gbs"] = out["roofline"]["hbm_gbs"]
        out["roofline"]["counters_source"] = os.path.relpath(path, HERE) if figs else None
    if not args.no_cpu_baseline:
        log("timing CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


def preroll(step, ms):
    """Untimed steps, in batches of 10 with a synchronisation after each, until `ms` of wall
    time have passed (clock ramp-up).  Returns (steps, seconds)."""
    import time

    import torch

    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        n += 10
    return n, time.perf_counter() - t0


def bench_tensor(args, wl):
    """The Tensor class's operations through the pybind module: host wall clock around
    synchronised batches of launches (the module's work runs on its own stream), outputs from
    the module's caching allocator (warm after the first call)."""
    import time

    import numpy as np
    from cudatransformer_amd import cuda_transformer as ctm

    n = 64 << 20
    rng = np.random.default_rng(3)
    a = ctm.FloatTensor.fromNumpy(rng.standard_normal(n, dtype=np.float32))
    b = ctm.FloatTensor.fromNumpy(rng.standard_normal(n, dtype=np.float32))
    sq = a.reshape([8192, 8192])
    ma = ctm.FloatTensor.fromNumpy(rng.standard_normal((4096, 4096), dtype=np.float32))
    mb = ctm.FloatTensor.fromNumpy(rng.standard_normal((4096, 4096), dtype=np.float32))

    def timed(fn, reps):
        for _ in range(max(args.warmup // 10, 2)):
            fn()
        ctm.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        ctm.synchronize()
        return (time.perf_counter() - t0) / reps

    reps = max(args.steps // 2, 10)
    t_add = timed(lambda: a + b, reps)
    t_sum = timed(lambda: a.sum(), reps)
    t_cast = timed(lambda: a.bfloat(), reps)
    t_tr = timed(lambda: sq.transpose(1, 0), reps)
    t_mm = timed(lambda: ma @ mb, max(reps // 2, 5))
    gbs = lambda nbytes, t: nbytes / t / 1e9
    add_gbs = gbs(3 * 4 * n, t_add)
    out = {
        "metric": wl["metric"], "value": round(add_gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": reps, "warmup": max(args.warmup // 10, 2), "ms_per_step": round(t_add * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": wl["label"],
                   "add_gbs": round(add_gbs, 1), "sum_gbs": round(gbs(4 * n, t_sum), 1),
                   "cast_bf16_gbs": round(gbs(6 * n, t_cast), 1), "transpose_gbs": round(gbs(8 * n, t_tr), 1),
                   "matmul_4096_tflops": round(2 * 4096 ** 3 / t_mm / 1e12, 1)},
        "roofline": {"bound": "hbm", "kernel": "binary_kernel<float, false> (a + b)", "achieved": round(add_gbs, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(add_gbs / 8000.0, 4), "traffic": None},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def time_layer_path(q, do, args):
    """ms per fwd+bwd step of the C++ FlashAttentionLayer through pybind, allocations included."""
    import time

    import torch
    from cudatransformer_amd import cuda_transformer as ctm

    g = torch.Generator(device=q.device).manual_seed(3)
    arrs = [torch.randn(q.shape, generator=g, device=q.device).cpu().numpy() for _ in range(3)]
    tq, tk, tv = (ctm.FloatTensor.fromNumpy(a) for a in arrs)
    tdo = ctm.FloatTensor.fromNumpy(do.float().cpu().numpy())
    layer = ctm.FlashAttention(D, H, CAUSAL)

    def step():
        layer.computeAttention(tq, tk, tv, True)
        layer.computeBackward(tq, tk, tv, tdo)

    for _ in range(args.warmup):
        step()
    ctm.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctm.synchronize()
    return (time.perf_counter() - t0) * 1e3 / args.steps


def bench_layer(args, wl):
    """The reference test's AttentionLayer (QKV projection -> attention -> output projection)
    through the C++ AttentionFloat layer (pybind): forward_caching + backward_caching per
    step, every output, gradient and workspace allocated by the layer as in real use; host
    wall clock around synchronised steps."""
    import time

    import numpy as np
    import torch
    from cudatransformer_amd import cuda_transformer as ctm

    b, h, n, d, e = wl["B"], wl["H"], wl["T"], wl["D"], wl["E"]
    hd = h * d
    rng = np.random.default_rng(12)
    suffix = "BFloat" if wl["dtype"] == "bf16" else "Float"
    tensor = getattr(ctm, suffix + "Tensor")
    layer = getattr(ctm, "Attention" + suffix)(input_dim=e, num_heads=h, head_dim=d)
    for part, shape, scale in (("Query", (hd, e), e), ("Key", (hd, e), e), ("Value", (hd, e), e),
                               ("Output", (e, hd), hd)):
        getattr(layer, f"set{part}Weights")(tensor.fromNumpy(
            (rng.standard_normal(shape) / np.sqrt(scale)).astype(np.float32)))
    x = tensor.fromNumpy(rng.standard_normal((b, n, e)).astype(np.float32))
    dy = tensor.fromNumpy(rng.standard_normal((b, n, e)).astype(np.float32))

    def fwd():
        return layer(x)

    def step():
        _, states = layer.forward_caching(x)
        layer.backward_caching(x, dy, states)

    def timed(fn, k):
        for _ in range(args.warmup):
            fn()
        ctm.synchronize()
        t0 = time.perf_counter()
        for _ in range(k):
            fn()
        ctm.synchronize()
        return (time.perf_counter() - t0) * 1e3 / k

    fwd_ms = timed(fwd, args.steps)
    ms = timed(step, args.steps)
    rows = b * n
    gemm = 2.0 * rows * hd * e
    attn_fwd = 4.0 * b * h * n * n * d
    fwd_flop = 4 * gemm + attn_fwd               # Q, K, V, output projections + attention
    step_flop = fwd_flop + 8 * gemm + 2.5 * attn_fwd  # + dW and dX of all four, attention bwd
    value = step_flop / (ms * 1e-3) / 1e12
    out = {
        "metric": wl["metric"], "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": wl["dtype"], "data": "synthetic",
        "pct_of_peak": round(100.0 * value / wl["peak"], 2),
        "config": {"workload": wl["label"], "B": b, "N": n, "E": e, "H": h, "d": d, "causal": False,
                   "step_gflop": round(step_flop / 1e9, 3), "fwd_ms": round(fwd_ms, 5),
                   "fwd_tflops": round(fwd_flop / (fwd_ms * 1e-3) / 1e12, 3)},
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_nanogpt(args, wl, dev):
    """Config 5: full training steps (forward, backward, Adam) of the NanoGPT host with its
    attention on the ctattn kernels; tokens/s and the losses of the timed steps."""
    import torch

    from cudatransformer_amd.nanogpt import (CONFIG5, NanoGPT, attention_flops_per_step, make_batch,
                                             model_flops_per_step, train_step)

    cfg = CONFIG5
    model = NanoGPT(**cfg, attention="ctattn").init_weights(5).to(dev)
    opt = torch.optim.Adam(model.parameters(), lr=cfg["lr"], betas=(0.9, 0.999), eps=1e-8)
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=5)
    ids, tgt = ids.to(dev), tgt.to(dev)
    for _ in range(args.warmup):
        train_step(model, opt, ids, tgt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    losses = [train_step(model, opt, ids, tgt) for _ in range(args.steps)]
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    tokens = cfg["batch"] * cfg["seq_len"]
    out = {
        "metric": wl["metric"], "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": wl["label"], "model_tflops": round(model_flops_per_step() / (ms * 1e-3) / 1e12, 2),
                   "attention_gflop_per_step": round(attention_flops_per_step() / 1e9, 3),
                   "loss_first": round(float(losses[0]), 4), "loss_last": round(float(losses[-1]), 4)},
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_native_nanogpt(args, wl):
    """Config 5 on the native host (cuda_transformer.FloatNanoGPT, every layer in
    libctattn.so): forward (probabilities), loss, zeroGrad, backward, Adam step.  The host
    orders all work on its own stream, so the timed region is bracketed by host clocks
    around that stream's synchronisation."""
    import time

    import numpy as np

    from cudatransformer_amd import cuda_transformer as ctm
    from cudatransformer_amd.nanogpt import (CONFIG5, NanoGPT, attention_flops_per_step, make_batch,
                                             model_flops_per_step, to_native)

    cfg = CONFIG5
    model = to_native(NanoGPT(**cfg, attention="sdpa").init_weights(5))
    opt = ctm.FloatAdamOptimizer(model.getParameters(), lr=cfg["lr"], b1=0.9, b2=0.999, eps=1e-8)
    ids, tgt = make_batch(cfg["batch"], cfg["seq_len"], cfg["vocab"], seed=5)
    ids = ctm.IntTensor.fromNumpy(ids.numpy().astype(np.int32))
    tgt = ctm.IntTensor.fromNumpy(tgt.numpy().astype(np.int32))

    def step():
        probs = model.forward(ids)
        loss = model.loss(probs, tgt)
        model.zeroGrad()
        model.backward(ids, probs, tgt)
        opt.step(model.getGradients())
        return loss

    for _ in range(args.warmup):
        step()
    ctm.synchronize()
    t0 = time.perf_counter()
    losses = [step() for _ in range(args.steps)]
    ctm.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    first, last = float(losses[0].numpy().sum()), float(losses[-1].numpy().sum())
    tokens = cfg["batch"] * cfg["seq_len"]
    out = {
        "metric": wl["metric"], "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": wl["label"], "model_tflops": round(model_flops_per_step() / (ms * 1e-3) / 1e12, 2),
                   "attention_gflop_per_step": round(attention_flops_per_step() / 1e9, 3),
                   "loss_first": round(first, 4), "loss_last": round(last, 4)},
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
