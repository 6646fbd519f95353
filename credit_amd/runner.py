"""Split / no-split sweep and cost-model scoring on one MI355X.

The gfx950 counterpart of the reference's evaluation runner
(dsmem_eval/runner.py:623-794, driven by scripts/run_local.py:82-100).  The
reference spawns one CUDA executable per (workload, cluster size) and parses
its stdout (runner.py:280-310); here every variant is an in-process call
through ``hip_lib.HIP_LAUNCHERS``:

* the block variants (READ, and STAGED where the row fits one workgroup)
  give ``block_ms`` -- the reference's best non-DSMEM time;
* SPLIT with P members for P in ``splits`` gives ``cluster_ms[P]``;
* ``credit_control_overhead`` gives the barrier cost for each (workload,
  N, P) -- the reference's cluster_control run -- with the barrier
  workgroups shaped like that split launch (its block size and LDS,
  ``credit_last_split_shape``), as the reference passes each point's
  staged slice as --shared-bytes;
* every variant's output is checked against the READ variant's (the
  reference never compared its CUDA kernels with anything).

``build_summary`` then scores the cost model exactly as the reference does
(runner.py:444-620): the predicted split factor is the one with the largest
predicted delta, ``measured_profitable`` is best split < block, and
``model_correct`` is their agreement.

    python -m credit_amd.runner --workloads all --output-dir results/local
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import platform
import statistics
import sys
import time
from collections import defaultdict
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch

from . import bundle, hip_lib
from .bundle import write_table
from .cost_model import (MODEL_VERSION, DeviceProfile, estimate, predict_traffic,
                         staged_bytes_per_workgroup)
from .profile import format_profile_text, make_device_profile, profile_as_dict, run_microbenchmarks
from .report import write_report
from .timing import run_trials
from .workloads import WORKLOADS, WorkloadSpec

# Workloads with a split variant (the cost model's domain).
SWEEP_WORKLOADS = (
    "row_sum_max",
    "layernorm_fwd",
    "rmsnorm_fwd",
    "rmsnorm_bwd",
    "softmax_fwd",
    "softmax_bwd",
    "softmax_logits_backward",
    "layernorm_backward",
    "layernorm_backward_bf16",
    "rowwise_quant",
    "lars_momentum",
    "weighted_var_backward",
    "pearson_backward",
)
DEFAULT_N_VALUES = (4096, 8192, 16384, 32768, 65536, 131072, 262144)
DEFAULT_SPLITS = (2, 4, 8, 16, 32)
# Rows per sweep point: as many as make one input tensor this large, so the
# rotating buffer sets (3 x inputs + outputs) exceed the 256 MB MALL and
# every point streams from HBM.
DEFAULT_TENSOR_BYTES = 256 << 20


@dataclass(frozen=True)
class RunConfig:
    """As dsmem_eval/runner.py:36-89 (cluster_sizes -> splits)."""

    workloads: tuple[str, ...] = SWEEP_WORKLOADS
    n_values: tuple[int, ...] = DEFAULT_N_VALUES
    splits: tuple[int, ...] = DEFAULT_SPLITS
    warmup: int = 5
    iterations: int = 20
    trials: int = 5
    quick: bool = False
    profile_only: bool = False
    tensor_bytes: int = DEFAULT_TENSOR_BYTES
    buffer_sets: int = 3
    settle_ms: float = 20.0

    @classmethod
    def from_dict(cls, raw: dict[str, Any]) -> "RunConfig":
        cfg = cls(
            workloads=tuple(raw.get("workloads", SWEEP_WORKLOADS)),
            n_values=tuple(int(v) for v in raw.get("n_values", DEFAULT_N_VALUES)),
            splits=tuple(int(v) for v in raw.get("splits", DEFAULT_SPLITS)),
            warmup=int(raw.get("warmup", 5)),
            iterations=int(raw.get("iterations", 20)),
            trials=int(raw.get("trials", 5)),
            quick=bool(raw.get("quick", False)),
            profile_only=bool(raw.get("profile_only", False)),
            tensor_bytes=int(raw.get("tensor_bytes", DEFAULT_TENSOR_BYTES)),
            buffer_sets=int(raw.get("buffer_sets", 3)),
            settle_ms=float(raw.get("settle_ms", 20.0)),
        )
        cfg.validate()
        return cfg

    def validate(self) -> None:
        unknown = sorted(set(self.workloads) - set(SWEEP_WORKLOADS))
        if unknown:
            raise ValueError(f"unknown sweep workloads: {', '.join(unknown)}")
        if not self.workloads and not self.profile_only:
            raise ValueError("at least one workload is required")
        if not self.n_values or any(v <= 0 for v in self.n_values):
            raise ValueError("n_values must contain positive integers")
        if not self.splits or any(v < 2 or v > 64 for v in self.splits):
            raise ValueError("splits must lie in [2, 64]")
        if min(self.warmup, self.iterations, self.trials, self.buffer_sets) <= 0:
            raise ValueError("warmup, iterations, trials and buffer_sets must be positive")

    def effective(self) -> "RunConfig":
        """Quick mode (runner.py:77-89): two widths, two splits, short timing,
        32 MiB tensors."""
        if not self.quick:
            return self
        return dataclasses.replace(self, n_values=self.n_values[:2], splits=self.splits[:2],
                                   warmup=2, iterations=5, trials=1, tensor_bytes=32 << 20)


# ---------------------------------------------------------------- sweep ----


def sweep_rows(spec: WorkloadSpec, cols: int, tensor_bytes: int) -> int:
    elem = 2 if spec.name in ("layernorm_fwd", "rmsnorm_fwd", "rmsnorm_bwd",
                              "layernorm_backward_bf16") else 4
    return int(max(tensor_bytes // (cols * elem), 8))


def variant_list(spec: WorkloadSpec, cols: int, splits: tuple[int, ...]):
    out = [("read", 0)]
    if cols <= spec.staged_max_cols:
        out.append(("staged", 0))
    out += [("split", p) for p in splits]
    return out


def _close(a: torch.Tensor, b: torch.Tensor) -> bool:
    if not a.is_floating_point():
        return bool(torch.equal(a, b))
    if a.dtype == torch.bfloat16:
        return bool(torch.allclose(a.float(), b.float(), rtol=1e-2, atol=1e-2, equal_nan=True))
    return bool(torch.allclose(a, b, rtol=1e-5, atol=1e-6, equal_nan=True))


def measure_point(name: str, spec: WorkloadSpec, rows: int, cols: int, cfg: RunConfig,
                  dev: torch.device) -> list[dict[str, Any]]:
    """Time every variant of one (workload, rows, cols) point."""
    cpu = spec.make_inputs(rows, cols, seed=1234 + cols)
    sets = [hip_lib.prepare_inputs(name, cpu, dev) for _ in range(cfg.buffer_sets)]
    outs = [hip_lib.allocate_outputs(name, ins) for ins in sets]
    launcher = hip_lib.HIP_LAUNCHERS[name]
    # Reference output from the READ variant for the cross-variant check.
    launcher(sets[0], outs[0], hip_lib.LaunchConfig("read", 0))
    torch.cuda.synchronize()
    reference = [o.clone() for o in outs[0]]
    results = []
    for variant, split in variant_list(spec, cols, cfg.splits):
        lc = hip_lib.LaunchConfig(variant, split)
        row = {"workload": name, "rows": rows, "cols": cols, "variant": variant, "split": split}
        try:
            for o in outs[0]:
                o.fill_(float("nan") if o.is_floating_point() else -128)
            launcher(sets[0], outs[0], lc)
            torch.cuda.synchronize()
            hip_lib.check_watchdog()
            row["correct"] = all(_close(o, r) for o, r in zip(outs[0], reference))
            if variant == "split":
                # The launch's own shape prices its control overhead
                # (runner.py:714-723 passes the staged slice as --shared-bytes).
                row.update(hip_lib.last_split_shape())
            # Arguments checked and converted once per buffer set: the timed
            # calls are the library calls alone, not the launcher's Python.
            bound = [hip_lib.bind(name, ins, o, lc) for ins, o in zip(sets, outs)]
            stats = run_trials(lambda i: bound[i % len(bound)](), cfg.trials, cfg.iterations,
                               cfg.warmup, cfg.settle_ms)
            hip_lib.check_watchdog()
            row.update(ms=stats.median_ms, p20_ms=stats.p20_ms, p80_ms=stats.p80_ms,
                       samples=stats.trials)
        except hip_lib.CreditError as err:
            row["error"] = f"{err.status}: {err}"
            row.update(ms=math.nan, p20_ms=math.nan, p80_ms=math.nan, samples=0)
        results.append(row)
    del sets, outs, reference
    torch.cuda.empty_cache()
    return results


def measure_control(rows: int, split: int, barriers: int, cfg: RunConfig, threads: int = 0,
                    lds_bytes: int = 0) -> float:
    """Median over trials of the barrier grid's time minus the plain grid's
    (runner.py:313-347), the barrier workgroups shaped like the split launch
    they price: `threads` lanes and `lds_bytes` of LDS."""
    samples = []
    for _ in range(cfg.trials):
        plain, coop = hip_lib.control_overhead(rows, split, max(barriers, 1), cfg.warmup,
                                               cfg.iterations, lds_bytes=lds_bytes,
                                               threads=threads)
        samples.append(max(coop - plain, 0.0))
    return statistics.median(samples)


# -------------------------------------------------------------- summary ----


def build_summary(raw: list[dict[str, Any]], control: dict[tuple[str, int, int], float],
                  profile: DeviceProfile, cfg: RunConfig):
    """summary and cluster_sweep rows (dsmem_eval/runner.py:444-620)."""
    by_point: dict[tuple[str, int, int], list[dict]] = defaultdict(list)
    for r in raw:
        by_point[(r["workload"], r["rows"], r["cols"])].append(r)
    summary, sweep = [], []
    for (name, rows, cols), rs in sorted(by_point.items()):
        spec = dataclasses.replace(WORKLOADS[name], rows=rows)
        blocks = [r for r in rs if r["variant"] in ("read", "staged") and math.isfinite(r["ms"])]
        splits = [r for r in rs if r["variant"] == "split" and math.isfinite(r["ms"])]
        if not blocks or not splits:
            continue
        block = min(blocks, key=lambda r: r["ms"])
        best_split = min(splits, key=lambda r: r["ms"])
        candidates = []
        for r in splits:
            ctl = control.get((name, cols, r["split"]), math.nan)
            if not math.isfinite(ctl):
                continue
            m = estimate(spec, cols, r["split"], ctl, profile, baseline_ms=block["ms"], rows=rows)
            tp = predict_traffic(spec, cols, r["split"], profile, rows=rows)
            candidates.append((m.predicted_delta_ms, r["split"], m))
            sweep.append({
                "workload": name, "rows": rows, "cols": cols, "split": r["split"],
                "staged_bytes_per_workgroup": staged_bytes_per_workgroup(spec, cols, r["split"]),
                "split_ms": r["ms"], "split_p20_ms": r["p20_ms"], "split_p80_ms": r["p80_ms"],
                "control_overhead_ms": ctl, "model_version": MODEL_VERSION,
                **{k: v for k, v in asdict(m).items()},
                "measured_delta_vs_block_ms": block["ms"] - r["ms"],
                "measured_profitable_vs_block": r["ms"] < block["ms"],
                "predicted_hbm_bytes": tp.hbm_bytes,
                "predicted_block_hbm_bytes": tp.block_hbm_bytes,
                "predicted_l2_requests": tp.l2_requests, "predicted_lds_bytes": tp.lds_bytes,
            })
        if not candidates:
            continue
        pred_delta, pred_split, pred = max(candidates, key=lambda c: c[0])
        measured_profitable = best_split["ms"] < block["ms"]
        summary.append({
            "workload": name, "label": spec.label, "category": spec.category,
            "rows": rows, "cols": cols,
            "block_variant": block["variant"], "block_ms": block["ms"],
            "block_p20_ms": block["p20_ms"], "block_p80_ms": block["p80_ms"],
            "split_ms": best_split["ms"], "measured_split": best_split["split"],
            "split_vs_block": block["ms"] / best_split["ms"],
            "block_gbps": spec.algorithmic_bytes(rows, cols) / (block["ms"] * 1e6),
            "split_gbps": spec.algorithmic_bytes(rows, cols) / (best_split["ms"] * 1e6),
            "predicted_split": pred_split, "model_version": MODEL_VERSION,
            "predicted_delta_ms": pred_delta,
            "predicted_profitable": pred.predicted_profitable,
            "measured_profitable": measured_profitable,
            "model_correct": pred.predicted_profitable == measured_profitable,
            "all_variants_correct": all(r.get("correct", True) for r in rs if "error" not in r),
        })
    return summary, sweep


def aggregate(summary: list[dict[str, Any]]) -> dict[str, Any]:
    n = len(summary)
    ok = sum(1 for r in summary if r["model_correct"])
    return {"points": n, "model_correct": ok, "model_accuracy": ok / n if n else math.nan,
            "split_profitable_points": sum(1 for r in summary if r["measured_profitable"]),
            "all_variants_correct": all(r["all_variants_correct"] for r in summary)}


def run_suite(raw_config: dict[str, Any], output_dir: Path,
              profile_text: str | None = None) -> dict[str, Any]:
    """As dsmem_eval/runner.py:623-794: calibrate, sweep, score, write the
    bundle (metadata.json, primitive_profile.json, raw.csv, control.csv,
    summary.csv, cluster_sweep.csv)."""
    if not torch.cuda.is_available():
        raise RuntimeError("a GPU is required")
    cfg = RunConfig.from_dict(raw_config).effective()
    output_dir.mkdir(parents=True, exist_ok=True)
    dev = torch.device("cuda:0")
    started = time.time()
    hip_lib.load_library()
    info = hip_lib.query_device(0)
    metadata: dict[str, Any] = {
        "status": "running", "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "device": info["name"], "arch": info["arch"], "cus": info["cu_count"],
        "torch_version": torch.__version__, "hip_version": torch.version.hip,
        "library": hip_lib.load_library().credit_version().decode(),
        "cost_model": {"version": MODEL_VERSION,
                       "baseline_calibration": "best no-split (READ/STAGED) time at the same shape"},
        "python_version": platform.python_version(), "config": asdict(cfg),
    }
    (output_dir / "metadata.json").write_text(json.dumps(metadata, indent=2) + "\n")
    if profile_text is None:
        parsed = run_microbenchmarks()
        profile_text = format_profile_text(parsed)
    from .profile import parse_profile_text

    parsed = parse_profile_text(profile_text)
    profile = make_device_profile(parsed)
    (output_dir / "primitive_stdout.txt").write_text(profile_text)
    (output_dir / "primitive_profile.json").write_text(json.dumps(
        {"measurements": parsed, "cost_model_profile": profile_as_dict(profile)}, indent=2) + "\n")
    if cfg.profile_only:
        metadata.update(status="complete", elapsed_seconds=time.time() - started)
        (output_dir / "metadata.json").write_text(json.dumps(metadata, indent=2) + "\n")
        return metadata

    raw: list[dict[str, Any]] = []
    control: dict[tuple[str, int, int], float] = {}
    control_rows: list[dict[str, Any]] = []
    lds_per_cu = int(info["lds_bytes_per_cu"])
    for name in cfg.workloads:
        spec = WORKLOADS[name]
        for cols in cfg.n_values:
            rows = sweep_rows(spec, cols, cfg.tensor_bytes)
            print(f"sweep {name}: rows={rows} cols={cols}", flush=True)
            point = measure_point(name, spec, rows, cols, cfg, dev)
            raw += point
            # One control run per (workload, N, P), shaped like that split
            # launch (runner.py:692-723 keys its control samples the same way).
            for r in point:
                if r["variant"] != "split" or "threads" not in r:
                    continue
                lds = hip_lib.control_lds_bytes(r, lds_per_cu)
                key = (name, cols, r["split"])
                control[key] = measure_control(rows, r["split"], spec.barrier_count, cfg,
                                               threads=r["threads"], lds_bytes=lds)
                control_rows.append({"workload": name, "cols": cols, "rows": rows,
                                     "split": r["split"], "barriers": spec.barrier_count,
                                     "threads": r["threads"], "lds_bytes": lds,
                                     "per_cu": r["per_cu"], "overhead_ms": control[key]})
            write_table(output_dir / "raw.csv", raw, bundle.RAW)
    write_table(output_dir / "control.csv", control_rows, bundle.CONTROL)
    summary, sweep = build_summary(raw, control, profile, cfg)
    write_table(output_dir / "summary.csv", summary, bundle.SUMMARY)
    write_table(output_dir / "cluster_sweep.csv", sweep, bundle.SWEEP)
    metadata.update(status="complete", elapsed_seconds=time.time() - started,
                    profile=profile_as_dict(profile), aggregate=aggregate(summary))
    metadata["report"] = write_report(output_dir, summary, metadata)
    (output_dir / "metadata.json").write_text(json.dumps(metadata, indent=2) + "\n")
    return metadata


def main(argv=None) -> int:
    """The run_local.py equivalent (scripts/run_local.py:49-100)."""
    def ints(v: str) -> tuple[int, ...]:
        return tuple(int(x) for x in v.split(",") if x.strip())

    ap = argparse.ArgumentParser(description="split-row sweep and cost-model scoring (gfx950)")
    ap.add_argument("--workloads", default="all",
                    help=f"comma list or 'all' ({', '.join(SWEEP_WORKLOADS)})")
    ap.add_argument("--n-values", type=ints, default=DEFAULT_N_VALUES)
    ap.add_argument("--splits", type=ints, default=DEFAULT_SPLITS)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iterations", type=int, default=20)
    ap.add_argument("--trials", type=int, default=5)
    ap.add_argument("--settle-ms", type=float, default=20.0,
                    help="wall time each variant runs before its warmup calls")
    ap.add_argument("--tensor-bytes", type=int, default=DEFAULT_TENSOR_BYTES,
                    help="rows per point: as many as make one input tensor this large")
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--profile-only", action="store_true")
    ap.add_argument("--profile-text", type=Path,
                    help="reuse a saved calibration (credit_amd.profile output)")
    ap.add_argument("--output-dir", type=Path,
                    default=Path("results") / datetime.now(timezone.utc).strftime("local_%Y%m%dT%H%M%SZ"))
    args = ap.parse_args(argv)
    workloads = SWEEP_WORKLOADS if args.workloads == "all" else tuple(
        w.strip() for w in args.workloads.split(",") if w.strip())
    config = {"workloads": workloads, "n_values": args.n_values, "splits": args.splits,
              "warmup": args.warmup, "iterations": args.iterations, "trials": args.trials,
              "settle_ms": args.settle_ms, "quick": args.quick, "profile_only": args.profile_only,
              "tensor_bytes": args.tensor_bytes}
    text = args.profile_text.read_text() if args.profile_text else None
    meta = run_suite(config, args.output_dir.resolve(), text)
    print(f"Status: {meta['status']}")
    print(f"Results: {args.output_dir}")
    if "aggregate" in meta:
        print(json.dumps(meta["aggregate"]))
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
