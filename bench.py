#!/usr/bin/env python3
"""Benchmark of the wide-row kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one call of the hot path over one batch of synthetic input (the
BASELINE configuration's full shape, inputs from a seeded CPU generator,
already resident in HBM).  The headline workload is BASELINE configs[1]
(LayerNorm forward, bf16 2048 x 32768); every other built configuration is
measured the same way and reported under "suite".  Per workload:

* inputs and outputs rotate through --sets buffer sets, so the 256 MB
  Infinity Cache cannot serve a repeated working set;
* --settle-ms of back-to-back calls first (after an idle period the MI355X
  takes 10-20 ms of sustained HBM traffic to reach its settled rate), then
  W warmup steps;
* the contract's timed region: exactly K steps bracketed by a device
  synchronisation on both sides, HIP events on the launch stream inside it:
  ``ms_per_step`` (wall) and ``kernel_ms`` (events), from which ``value``
  and ``roofline.achieved`` come;
* then --trials blocks of max(20, K) steps: ``trials`` holds the median and
  the 20th / 80th percentiles of the per-step event time;
* the split-row watchdog is checked after the timed calls; a barrier that
  gave up waiting fails the run (exit 3) instead of reporting a time;
* ``roofline.ceiling``: the library's own settled HBM stream kernels
  (credit_stream_ceiling) at the workload's read:write byte mix and call
  size, over the same number of rotating sets; ``frac`` of it is reported
  beside the fraction of the 8 TB/s peak;
  for the FFN, the attainable dense bf16 MFMA rate (back-to-back MFMA
  chains on every CU, no memory traffic) and the shader clock it ran at;
* ``roofline.traffic``: HBM bytes per call from the committed rocprofv3 PMC
  summary, or null when the kernels' sources changed after it was taken;
* ``cpu_baseline``: the reference's PyTorch path on the host cores.

Each step is one library call whose arguments were checked and converted
once (hip_lib.bind), so a short kernel is not timed behind its Python
checks.  Prints ONE JSON line (each suite entry in compact form; every
workload's full record goes to --detail).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# Workloads whose tensors are bf16 (fp32 accumulation); the rest compute in fp32.
BF16_WORKLOADS = ("layernorm_fwd", "rmsnorm_fwd", "rmsnorm_bwd", "ffn", "ffn_baseline_layout",
                  "ffn_backward", "ffn_backward_saved", "ffn_backward_baseline_layout",
                  "layernorm_backward_bf16")
FFN_WORKLOADS = ("ffn", "ffn_baseline_layout", "ffn_backward", "ffn_backward_saved",
                 "ffn_backward_baseline_layout")

# Kernels one AUTO call launches at the BASELINE shape (names as rocprofv3
# reports them) and the source file they are built from; the committed PMC
# summary (FETCH_SIZE / WRITE_SIZE, scaled by a stream kernel of known size;
# credit_amd/traffic.py) gives their HBM bytes per call while that source
# still hashes as it did when the counters were taken.
TRAFFIC_SUMMARY = ROOT / "profiles" / "hbm_traffic_suite.json"
CALL_KERNELS = {
    "row_sum_max": ("rowreduce.hip", ["row_sum_max_read_kernel<256>"]),
    "layernorm_fwd": ("layernorm.hip", ["layernorm_fwd_pipe_kernel<512, 8>"]),
    "rmsnorm_fwd": ("rmsnorm.hip", ["rmsnorm_fwd_group_kernel<512, 4, 4, 1>"]),
    "rmsnorm_bwd": ("rmsnorm.hip", ["rmsnorm_bwd_group_kernel<512, 2, 4, 2>",
                                    "rmsnorm_dw_reduce_kernel"]),
    "rmsnorm_fwd_bwd": ("rmsnorm.hip", ["rmsnorm_fused_group_kernel<512, 2, 2, 2>",
                                        "rmsnorm_dw_reduce_kernel"]),
    "softmax_fwd": ("softmax.hip", ["softmax_fwd_group_kernel<512, 8, true>"]),
    "softmax_bwd": ("softmax.hip", ["softmax_bwd_group_kernel<512, 4, true>"]),
    "softmax_logits_backward": ("softmax.hip", ["softmax_logits_bwd_slice_kernel<1024, 8>"]),
    "ffn": ("ffn.hip", ["ffn_rstd_kernel", "ffn_gemm256_kernel<0, false>",
                        "ffn_gemm256_kernel<1, false>"]),
    "ffn_baseline_layout": ("ffn.hip", ["ffn_rstd_kernel", "ffn_gemm256_kernel<0, true>",
                                        "ffn_gemm256_kernel<1, true>"]),
    "layernorm_backward": ("lnbwd.hip", ["layernorm_bwd_slice_kernel<float, 1024, 8>"]),
    "layernorm_backward_bf16": ("lnbwd.hip", ["layernorm_bwd_group_kernel<512, 2, 4, 2>"]),
    "rowwise_quant": ("quant.hip", ["rowwise_quant_slice_kernel<1024, 16>"]),
    "lars_momentum": ("lars.hip", ["lars_slice_kernel<512, 8>"]),
    "weighted_var_backward": ("wvar.hip", ["wvar_bwd_slice_kernel<1024, 4>"]),
    "pearson_backward": ("pearson.hip", ["pearson_bwd_slice_kernel<512, 8>"]),
}


def measured_traffic(name):
    """(HBM bytes per call, note): bytes from the PMC summary, or None with
    the reason when there is no current figure."""
    from credit_amd.traffic import sources_unchanged

    try:
        summary = json.loads(TRAFFIC_SUMMARY.read_text())
    except (OSError, ValueError):
        return None, "no PMC summary"
    source, kernels = CALL_KERNELS.get(name, (None, []))
    if source is None:
        return None, "no kernel map"
    if not sources_unchanged(summary.get("sources", {}), source):
        return None, f"stale: {source} changed after the PMC run at {summary.get('commit')}"
    try:
        return sum(summary["kernels"][k]["fetch_bytes"] + summary["kernels"][k]["write_bytes"]
                   for k in kernels), f"PMC at {summary.get('commit')}"
    except KeyError as err:
        return None, f"kernel {err} not in the PMC summary"


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--trials", type=int, default=5,
                    help="timed blocks of max(20, steps) steps for the median/p20/p80")
    ap.add_argument("--workload", default="layernorm_fwd")
    ap.add_argument("--suite", default="all",
                    help="comma list of extra workloads to measure, 'all' or 'none'")
    ap.add_argument("--sets", type=int, default=3, help="rotating buffer sets")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="wall time the workload runs before its warmup steps (HBM clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the stream-ceiling leg")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the per-variant sweep")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the CPU-baseline sample per workload")
    ap.add_argument("--detail", default="gpurun_out/bench_detail.json",
                    help="file for every workload's full record (variant sweep, ceilings, "
                         "trials); '' to skip")
    return ap.parse_args(argv)


class WatchdogTripped(RuntimeError):
    pass


# ----------------------------------------------------------- GPU timing ---


def build_case(name, spec, hip_lib, torch, dev, nsets):
    """Inputs (resident), rotating output sets and a launch(index, variant,
    split) issuing one bound library call on set index % nsets."""
    cpu_inputs = spec.make_inputs()
    inputs = [hip_lib.prepare_inputs(name, cpu_inputs, dev) for _ in range(nsets)]
    outputs = [hip_lib.allocate_outputs(name, ins) for ins in inputs]
    torch.cuda.synchronize()
    bound = {}

    def launch(i, variant="auto", split=0):
        key = (i % nsets, variant, split)
        if key not in bound:
            bound[key] = hip_lib.bind(name, inputs[key[0]], outputs[key[0]],
                                      hip_lib.LaunchConfig(variant, split))
        bound[key]()

    return cpu_inputs, launch


def check_watchdog(hip_lib, name, what):
    try:
        hip_lib.check_watchdog()
    except hip_lib.CreditError as err:
        raise WatchdogTripped(f"{name} ({what}): {err}") from err


def time_workload(name, launch, hip_lib, args):
    """Contract block of exactly K steps, then the trial blocks."""
    from credit_amd.timing import run_trials, settle, timed_block

    i = settle(launch, args.settle_ms)
    for _ in range(args.warmup):
        launch(i)
        i += 1
    ms_step, kernel_ms = timed_block(launch, args.steps, i)
    i += args.steps
    check_watchdog(hip_lib, name, "timed steps")
    trials = run_trials(launch, args.trials, max(20, args.steps), start=i)
    check_watchdog(hip_lib, name, "trials")
    return ms_step, kernel_ms, trials


# ----------------------------------------------------------- CPU baseline --


def host_threads():
    """(threads, affinity cores, cgroup CPU quota or None): every core this
    process may run on, capped by the cgroup's CPU quota when one is set
    (more threads than the quota only time-slice)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, -(-int(q) // int(period)))
    except (OSError, ValueError):
        quota = None
    return (min(affinity, quota) if quota else affinity), affinity, quota


def cpu_baseline(name, cpu_inputs, spec, seconds):
    """Time the reference's PyTorch path on the host cores (bounded sample)."""
    import torch

    from oracle import torch_cpu

    threads, affinity, quota = host_threads()
    torch.set_num_threads(threads)
    rows = cpu_inputs[0].shape[0]
    fn = torch_cpu.FUNCTIONS[name]
    args = tuple(cpu_inputs)
    if name == "rmsnorm_bwd":
        rstd = torch_cpu.rmsnorm_fwd(args[0], args[1])[1]
        fn, args = (lambda x, w, dy, r: torch_cpu.rmsnorm_bwd(x, w, dy, r)), (args[0], args[1], args[2], rstd)
    elif name == "softmax_bwd":
        p = torch.softmax(args[0], dim=-1)
        fn, args = torch_cpu.softmax_bwd, (p, args[1])
    elif name == "ffn_backward_saved":
        # the forward (with its saved activations) outside the timed calls
        fn, args = torch_cpu.ffn_backward_saved(*args), ()
    # Row sample: shrink the batch until one call takes <= seconds/4.
    sample_rows = rows
    t0 = time.perf_counter()
    fn(*args)
    one = time.perf_counter() - t0
    while one > seconds / 4 and sample_rows > 8 and name not in FFN_WORKLOADS:
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
    if name in FFN_WORKLOADS:
        work = spec_ffn_flops(sample_rows, cpu_inputs[0].shape[1], name)
        value, unit = work / med / 1e12, "TFLOP/s"
    else:
        work = spec.algorithmic_bytes(sample_rows, cpu_inputs[0].shape[1])
        value, unit = work / med / 1e9, "GB/s"
    return {
        "value": round(value, 3),
        "unit": unit,
        "cores": threads,
        "affinity_cores": affinity,
        "cgroup_cpu_quota": quota,
        "kind": "port",
        "sample": f"{sample_rows} of {rows} rows x {cpu_inputs[0].shape[1]} cols, median of {len(runs)} runs",
    }


def spec_ffn_flops(rows, d, name="ffn"):
    from credit_amd.workloads import ffn_backward_flops, ffn_flops

    return (ffn_backward_flops(rows, d) if name.startswith("ffn_backward")
            else ffn_flops(rows, d))


# ------------------------------------------------------------------ main --


def stream_ceiling(spec, nbytes, hip_lib, args):
    reads, writes = spec.stream_mix
    if reads + writes == 0:
        return None
    try:
        c = hip_lib.stream_ceiling(reads, writes, nbytes, trials=args.trials,
                                   iters=max(20, args.steps // 5), settle_ms=20.0)
    except hip_lib.CreditError as err:
        return {"mix": f"{reads}:{writes}", "error": str(err)}
    return c


def measure(name, args, hip_lib, torch, dev, with_cpu):
    from credit_amd.timing import run_trials
    from credit_amd.workloads import WORKLOADS

    spec = WORKLOADS[name]
    cpu_inputs, launch = build_case(name, spec, hip_lib, torch, dev, args.sets)
    ms_step, kernel_ms, trials = time_workload(name, launch, hip_lib, args)
    traffic, traffic_note = measured_traffic(name)
    out = {"rows": spec.rows, "cols": spec.cols, "ms_per_step": round(ms_step, 6),
           "kernel_ms": round(kernel_ms, 6), "trials": trials.as_dict(), "watchdog": "ok"}
    if name in FFN_WORKLOADS:
        flops = spec_ffn_flops(spec.rows, spec.cols, name)
        achieved = flops / (kernel_ms * 1e-3) / 1e12
        out.update(metric="MFMA TFLOP/s", value=round(flops / (ms_step * 1e-3) / 1e12, 2),
                   unit="TFLOP/s",
                   roofline={"bound": "mfma", "achieved": round(achieved, 2),
                             "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                             "frac_median": round(flops / (trials.median_ms * 1e-3) / 1e12
                                                  / BF16_PEAK_TFLOPS, 4),
                             "traffic": traffic, "traffic_source": traffic_note})
        # The shader clock the GEMM tiles ran at, over the same number of
        # settled calls as one trial block (the clock probe's stamps).
        i0 = 10 ** 6
        out["clock_MHz"] = round(hip_lib.gemm_clock_mhz(
            lambda: [launch(i0 + k) for k in range(max(20, args.steps))]), 1)
        if not args.no_ceiling:
            try:
                ceiling = hip_lib.mfma_ceiling()
                ceiling["frac"] = round(achieved / ceiling["TFLOPs"], 4)
            except hip_lib.CreditError as err:
                ceiling = {"error": str(err)}
            out["roofline"]["ceiling"] = ceiling
    else:
        nbytes = spec.algorithmic_bytes(spec.rows, spec.cols)
        achieved = nbytes / (kernel_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "frac_median": round(nbytes / (trials.median_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                "traffic": traffic, "traffic_source": traffic_note}
        if not args.no_ceiling:
            ceiling = stream_ceiling(spec, nbytes, hip_lib, args)
            if ceiling is not None and "GBps" in ceiling and ceiling["GBps"] > 0:
                ceiling["frac"] = round(achieved / ceiling["GBps"], 4)
            roof["ceiling"] = ceiling
        out.update(metric="HBM GB/s", value=round(nbytes / (ms_step * 1e-3) / 1e9, 1), unit="GB/s",
                   bytes_per_call=nbytes, roofline=roof)
        variants = {}
        for variant, split in ([] if args.no_variants else VARIANT_SWEEP.get(name, [])):
            label = f"{variant}{split or ''}"
            try:
                call = (lambda v, p: lambda i: launch(i, v, p))(variant, split)
                t = run_trials(call, 3, max(10, args.steps // 4), warmup=3,
                               settle_ms=args.settle_ms / 4)
                check_watchdog(hip_lib, name, f"variant {label}")
                variants[label] = round(nbytes / (t.median_ms * 1e-3) / 1e9, 1)
            except hip_lib.CreditError as err:
                variants[label] = f"unsupported: {err.status}"
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


def compact(entry):
    """A suite entry as it goes into the printed line: time, rate, roofline
    fractions, counted traffic over algorithmic bytes and the CPU baseline;
    the variant sweep and the full ceiling and trial records go to the
    detail file."""
    roof = entry["roofline"]
    ceiling = roof.get("ceiling") or {}
    out = {"ms": entry["kernel_ms"], "value": entry["value"], "unit": entry["unit"],
           "frac": roof["frac"], "frac_median": roof["frac_median"],
           "ceiling_frac": ceiling.get("frac")}
    if roof["bound"] == "hbm":
        out["traffic_ratio"] = (round(roof["traffic"] / entry["bytes_per_call"], 3)
                                if roof.get("traffic") else None)
    else:
        out["clock_MHz"] = entry.get("clock_MHz")
        out["mfma_chain_TFLOPs"] = ceiling.get("TFLOPs")
    cpu = entry.get("cpu_baseline")
    if cpu:
        out["cpu"] = {"value": cpu["value"], "unit": cpu["unit"], "cores": cpu["cores"]}
    return out


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (every box here has one); "
                                   "--gpus must be 1", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.steps < 1 or args.trials < 1 or args.warmup < 0:
        print(json.dumps({"error": "--steps and --trials must be >= 1, --warmup >= 0"}))
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

    try:
        head = measure(args.workload, args, hip_lib, torch, dev, not args.no_cpu_baseline)
        suite = {}
        if args.suite != "none":
            names = list(hip_lib.HIP_LAUNCHERS) if args.suite == "all" else args.suite.split(",")
            for name in names:
                if name == args.workload:
                    continue
                print(f"# bench {name}", file=sys.stderr, flush=True)
                suite[name] = measure(name, args, hip_lib, torch, dev, not args.no_cpu_baseline)
    except WatchdogTripped as err:
        print(json.dumps({"error": f"split-row watchdog expired: {err}", "watchdog": "tripped",
                          "n_gpus": 1}), flush=True)
        sys.exit(3)

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
        "kernel_ms": head["kernel_ms"],
        "trials": head["trials"],
        "watchdog": head["watchdog"],
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "suite": {name: compact(entry) for name, entry in suite.items()},
    }
    if args.detail:
        detail = Path(args.detail)
        if not detail.is_absolute():
            detail = ROOT / detail
        try:
            detail.parent.mkdir(parents=True, exist_ok=True)
            detail.write_text(json.dumps({"head": {args.workload: head}, "suite": suite},
                                         indent=1) + "\n")
            line["detail"] = str(detail.relative_to(ROOT)) if detail.is_relative_to(ROOT) \
                else str(detail)
        except OSError as err:
            line["detail"] = f"not written: {err}"
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
