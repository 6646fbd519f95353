#!/usr/bin/env python3
"""Benchmark of the wide-row kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one call of the hot path over one batch of synthetic input (the
BASELINE configuration's full shape, inputs from a seeded CPU generator,
already resident in HBM).  The headline workload is BASELINE configs[1]
(LayerNorm forward, bf16 2048 x 32768); every other built configuration is
measured the same way and reported under "suite".  Timing rotates through
several input/output buffer sets so the 256 MB Infinity Cache cannot serve a
repeated working set.  Before its W warmup steps each timed workload runs for
--settle-ms of wall time (default 100 ms): after an idle period the MI355X
takes 10-20 ms of sustained HBM traffic to reach its settled rate, and the K
timed steps measure that rate.  Each step is one library call whose arguments
were checked and converted once (hip_lib.bind), so a short kernel is not
timed behind its Python checks.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# Workloads whose tensors are bf16 (fp32 accumulation); the rest compute in fp32.
BF16_WORKLOADS = ("layernorm_fwd", "rmsnorm_fwd", "rmsnorm_bwd", "ffn", "ffn_backward",
                  "layernorm_backward_bf16")

# Kernels one AUTO call launches at the BASELINE shape, and the committed
# rocprofv3 PMC summary (FETCH_SIZE / WRITE_SIZE, scaled by a copy kernel of
# known size; credit_amd/traffic.py) their HBM bytes per call come from.
TRAFFIC_SUMMARY = ROOT / "profiles" / "hbm_traffic_suite.json"
CALL_KERNELS = {
    "row_sum_max": ["row_sum_max_read_kernel<256>"],
    "layernorm_fwd": ["layernorm_fwd_staged_kernel<512, 8>"],
    "rmsnorm_fwd": ["rmsnorm_fwd_slice_kernel<1024, 8>"],
    "rmsnorm_bwd": ["rmsnorm_bwd_group_kernel<512, 2>", "rmsnorm_dw_reduce_kernel"],
    "softmax_fwd": ["softmax_fwd_group_kernel<512, 8>"],
    "softmax_bwd": ["softmax_bwd_slice_kernel<512, 8>"],
    "softmax_logits_backward": ["softmax_logits_bwd_slice_kernel<1024, 8>"],
    "ffn": ["ffn_rstd_kernel", "ffn_gemm256_kernel<0>", "ffn_gemm256_kernel<1>"],
    "layernorm_backward": ["layernorm_bwd_slice_kernel<float, 1024, 8>"],
    "layernorm_backward_bf16": ["layernorm_bwd_slice_kernel<unsigned short, 512, 8>"],
    "rowwise_quant": ["rowwise_quant_slice_kernel<1024, 16>"],
    "lars_momentum": ["lars_slice_kernel<512, 8>"],
    "weighted_var_backward": ["wvar_bwd_slice_kernel<1024, 4>"],
    "pearson_backward": ["pearson_bwd_slice_kernel<512, 8>"],
}


def measured_traffic(name):
    """HBM bytes per call from the PMC summary, or None when not profiled."""
    try:
        kernels = json.loads(TRAFFIC_SUMMARY.read_text())["kernels"]
        return sum(kernels[k]["fetch_bytes"] + kernels[k]["write_bytes"]
                   for k in CALL_KERNELS[name])
    except (OSError, KeyError, ValueError):
        return None


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="layernorm_fwd")
    ap.add_argument("--suite", default="all",
                    help="comma list of extra workloads to measure, 'all' or 'none'")
    ap.add_argument("--sets", type=int, default=3, help="rotating buffer sets")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="wall time the workload runs before its warmup steps (HBM clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the CPU-baseline sample per workload")
    return ap.parse_args(argv)


# ----------------------------------------------------------- GPU timing ---


def build_case(name, spec, hip_lib, torch, dev, nsets):
    """Inputs (resident), rotating output sets and a launch(set_index, variant, split)."""
    cpu_inputs = spec.make_inputs()
    inputs = [hip_lib.prepare_inputs(name, cpu_inputs, dev) for _ in range(nsets)]
    outputs = [hip_lib.allocate_outputs(name, ins) for ins in inputs]
    torch.cuda.synchronize()
    bound = {}

    def launch(i, variant="auto", split=0):
        # Arguments are checked and converted once per (set, variant, split):
        # the timed loop then issues only the library calls.
        key = (i % nsets, variant, split)
        if key not in bound:
            bound[key] = hip_lib.bind(name, inputs[key[0]], outputs[key[0]],
                                      hip_lib.LaunchConfig(variant, split))
        bound[key]()

    return cpu_inputs, launch


def settle(launch, torch, settle_ms, variant="auto", split=0):
    """Run the workload for settle_ms of wall time, synchronising every 8
    calls so that wall time is GPU time.  After an idle period the first
    10-20 ms of HBM-bound work on the MI355X run up to 35% slower (measured
    per 100-call block: LayerNorm forward C2 65 -> 47.4 us per call); the
    timed steps measure the settled rate."""
    t_end = time.perf_counter() + settle_ms / 1e3
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            launch(i, variant, split)
            i += 1
        torch.cuda.synchronize()


def time_gpu(launch, torch, steps, warmup, variant="auto", split=0, settle_ms=0.0):
    if settle_ms > 0:
        settle(launch, torch, settle_ms, variant, split)
    for i in range(warmup):
        launch(i, variant, split)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        launch(i, variant, split)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall * 1e3 / steps, start.elapsed_time(stop) / steps


# ----------------------------------------------------------- CPU baseline --


def cpu_baseline(name, cpu_inputs, spec, seconds):
    """Time the reference's PyTorch path on the host cores (bounded sample)."""
    import torch

    from oracle import torch_cpu

    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    torch.set_num_threads(cores)
    rows = cpu_inputs[0].shape[0]
    fn = torch_cpu.FUNCTIONS[name]
    args = tuple(cpu_inputs)
    if name == "rmsnorm_bwd":
        rstd = torch_cpu.rmsnorm_fwd(args[0], args[1])[1]
        fn, args = (lambda x, w, dy, r: torch_cpu.rmsnorm_bwd(x, w, dy, r)), (args[0], args[1], args[2], rstd)
    elif name == "softmax_bwd":
        p = torch.softmax(args[0], dim=-1)
        fn, args = torch_cpu.softmax_bwd, (p, args[1])
    # Row sample: shrink the batch until one call takes <= seconds/4.
    sample_rows = rows
    t0 = time.perf_counter()
    fn(*args)
    one = time.perf_counter() - t0
    while one > seconds / 4 and sample_rows > 8 and name != "ffn":
        sample_rows //= 2
        args = tuple(a[:sample_rows] if a.dim() == 2 and a.shape[0] == rows else a for a in args)
        if name == "rmsnorm_bwd":
            args = args[:3] + (args[3][:sample_rows],)
        t0 = time.perf_counter()
        fn(*args)
        one = time.perf_counter() - t0
    runs = []
    deadline = time.perf_counter() + seconds
    while time.perf_counter() < deadline or len(runs) < 3:
        t0 = time.perf_counter()
        fn(*args)
        runs.append(time.perf_counter() - t0)
        if len(runs) >= 50:
            break
    runs.sort()
    med = runs[len(runs) // 2]
    if name in ("ffn", "ffn_backward"):
        work = spec_ffn_flops(sample_rows, cpu_inputs[0].shape[1], name)
        value, unit = work / med / 1e12, "TFLOP/s"
    else:
        work = spec.algorithmic_bytes(sample_rows, cpu_inputs[0].shape[1])
        value, unit = work / med / 1e9, "GB/s"
    return {
        "value": round(value, 3),
        "unit": unit,
        "cores": cores,
        "kind": "port",
        "sample": f"{sample_rows} of {rows} rows x {cpu_inputs[0].shape[1]} cols, median of {len(runs)} runs",
    }


def spec_ffn_flops(rows, d, name="ffn"):
    from credit_amd.workloads import ffn_backward_flops, ffn_flops

    return ffn_backward_flops(rows, d) if name == "ffn_backward" else ffn_flops(rows, d)


# ------------------------------------------------------------------ main --


def measure(name, args, hip_lib, torch, dev, with_cpu):
    from credit_amd.workloads import WORKLOADS

    spec = WORKLOADS[name]
    cpu_inputs, launch = build_case(name, spec, hip_lib, torch, dev, args.sets)
    ms_step, kernel_ms = time_gpu(launch, torch, args.steps, args.warmup, settle_ms=args.settle_ms)
    out = {"rows": spec.rows, "cols": spec.cols, "ms_per_step": round(ms_step, 6),
           "kernel_ms": round(kernel_ms, 6)}
    if name in ("ffn", "ffn_backward"):
        flops = spec_ffn_flops(spec.rows, spec.cols, name)
        out.update(metric="MFMA TFLOP/s", value=round(flops / (ms_step * 1e-3) / 1e12, 2),
                   unit="TFLOP/s",
                   roofline={"bound": "mfma", "achieved": round(flops / (kernel_ms * 1e-3) / 1e12, 2),
                             "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(flops / (kernel_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                             "traffic": measured_traffic(name)})
    else:
        nbytes = spec.algorithmic_bytes(spec.rows, spec.cols)
        achieved = nbytes / (kernel_ms * 1e-3) / 1e9
        out.update(metric="HBM GB/s", value=round(nbytes / (ms_step * 1e-3) / 1e9, 1), unit="GB/s",
                   bytes_per_call=nbytes,
                   roofline={"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                             "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                             "traffic": measured_traffic(name)})
        variants = {}
        for variant, split in VARIANT_SWEEP.get(name, []):
            try:
                _, vms = time_gpu(launch, torch, max(10, args.steps // 4), 3, variant, split,
                                  settle_ms=args.settle_ms / 4)
                variants[f"{variant}{split or ''}"] = round(nbytes / (vms * 1e-3) / 1e9, 1)
            except hip_lib.CreditError as err:
                variants[f"{variant}{split or ''}"] = f"unsupported: {err.status}"
        if variants:
            out["variants_GBps"] = variants
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(name, cpu_inputs, spec, args.cpu_seconds)
    del cpu_inputs
    torch.cuda.empty_cache()
    return out


VARIANT_SWEEP = {
    "row_sum_max": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "layernorm_fwd": [("read", 0), ("staged", 0)],
    "rmsnorm_fwd": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "rmsnorm_bwd": [("read", 0), ("split", 16), ("split", 18), ("split", 32), ("split", 37)],
    "softmax_fwd": [("read", 0), ("split", 4), ("split", 8), ("split", 16), ("split", 32)],
    "softmax_bwd": [("read", 0), ("split", 8), ("split", 16), ("split", 32)],
    "softmax_logits_backward": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "layernorm_backward": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "layernorm_backward_bf16": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "rowwise_quant": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "lars_momentum": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
    "weighted_var_backward": [("read", 0), ("split", 4), ("split", 8), ("split", 12)],
    "pearson_backward": [("read", 0), ("split", 2), ("split", 4), ("split", 8)],
}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from credit_amd import hip_lib

    if not hip_lib.LIB_PATH.is_file():
        import __graft_entry__

        __graft_entry__.build()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    hip_lib.load_library()
    info = hip_lib.query_device(0)

    head = measure(args.workload, args, hip_lib, torch, dev, not args.no_cpu_baseline)
    suite = {}
    if args.suite != "none":
        names = list(hip_lib.HIP_LAUNCHERS) if args.suite == "all" else args.suite.split(",")
        for name in names:
            if name == args.workload:
                continue
            print(f"# bench {name}", file=sys.stderr, flush=True)
            suite[name] = measure(name, args, hip_lib, torch, dev, not args.no_cpu_baseline)

    line = {
        "metric": "HBM GB/s (% of ~8 TB/s) on wide-row norms; MFMA TFLOPS on fused FFN",
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.workload in BF16_WORKLOADS else "f32",
        "data": "synthetic (seeded CPU generator, BASELINE distributions)",
        "config": {"workload": args.workload, "rows": head["rows"], "cols": head["cols"],
                   "device": info["name"], "arch": info["arch"], "cus": info["cu_count"],
                   "buffer_sets": args.sets},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "variants_GBps": head.get("variants_GBps"),
        "suite": suite,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
