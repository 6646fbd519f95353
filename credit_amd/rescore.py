"""Re-score saved split-sweep bundles with the current cost model.

    python -m credit_amd.rescore RUN_DIR [RUN_DIR ...] [--write]

The role of the reference's scripts/rescore_cost_model.py:99-218: a bundle
measured once on an MI355X is judged again, without a GPU, after the model
changes.  Everything the model needs was saved by the run: the calibrated
device profile (metadata.json "profile"), each split factor's measured
control overhead (cluster_sweep.csv) and each point's best no-split time
(summary.csv).  The measured side -- which variant won -- never changes;
only the prediction does.

A dry run reports the verdict counts before and after.  ``--write`` rewrites
summary.csv, cluster_sweep.csv (through credit_amd.bundle's typed schemas),
REPORT.md and the metadata's cost_model / aggregate fields, and appends one
JSON line to ``rescore_history.jsonl`` recording the model versions and every
point whose verdict changed, so the bundle keeps its own audit trail instead
of copies of the old tables.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

from .bundle import Bundle
from .cost_model import MODEL_VERSION, DeviceProfile, estimate, predict_traffic
from .report import render
from .workloads import WORKLOADS

HISTORY = "rescore_history.jsonl"

PointKey = tuple[str, int, int]


@dataclass(frozen=True)
class Rescore:
    run: str
    device: str
    points: int
    correct_before: int
    correct_after: int
    changed: tuple[dict[str, Any], ...]


def saved_profile(metadata: dict[str, Any]) -> DeviceProfile:
    """The calibrated profile a run stored in its metadata.json."""
    stored = metadata.get("profile")
    if not isinstance(stored, dict):
        raise ValueError("metadata.json carries no calibrated 'profile' (the run did not finish)")
    values = {}
    for f in dataclasses.fields(DeviceProfile):
        if f.name not in stored:
            raise ValueError(f"the saved profile lacks {f.name!r}")
        kind = {"str": str, "int": int, "float": float}[f.type if isinstance(f.type, str)
                                                         else f.type.__name__]
        values[f.name] = kind(stored[f.name])
    return DeviceProfile(**values)


def _key(row: dict[str, Any]) -> PointKey:
    return str(row["workload"]), int(row["rows"]), int(row["cols"])


def predict(bundle: Bundle, profile: DeviceProfile) -> dict[PointKey, dict[str, Any]]:
    """New model terms for every sweep row (updated in place) and, per
    point, the split factor with the largest predicted gain."""
    block_ms = {_key(r): float(r["block_ms"]) for r in bundle.summary}
    best: dict[PointKey, dict[str, Any]] = {}
    for row in bundle.sweep:
        key = _key(row)
        if key not in block_ms or not math.isfinite(block_ms[key]) or block_ms[key] <= 0:
            continue
        spec = dataclasses.replace(WORKLOADS[key[0]], rows=key[1])
        est = estimate(spec, key[2], int(row["split"]), float(row["control_overhead_ms"]),
                       profile, baseline_ms=block_ms[key], rows=key[1])
        tp = predict_traffic(spec, key[2], int(row["split"]), profile, rows=key[1])
        row.update(dataclasses.asdict(est), model_version=MODEL_VERSION,
                   predicted_hbm_bytes=tp.hbm_bytes, predicted_block_hbm_bytes=tp.block_hbm_bytes,
                   predicted_l2_requests=tp.l2_requests, predicted_lds_bytes=tp.lds_bytes)
        if key not in best or est.predicted_delta_ms > best[key]["predicted_delta_ms"]:
            best[key] = {"predicted_split": int(row["split"]),
                         "predicted_delta_ms": est.predicted_delta_ms,
                         "predicted_profitable": est.predicted_profitable}
    return best


def rescore(run: Path, write: bool = False) -> Rescore:
    bundle = Bundle.load(run)
    profile = saved_profile(bundle.metadata)
    before = {_key(r): r.get("model_correct") is True for r in bundle.summary}
    old_version = bundle.metadata.get("cost_model", {}).get("version")
    best = predict(bundle, profile)
    changed = []
    for row in bundle.summary:
        key = _key(row)
        if key not in best:
            continue
        row.update(best[key], model_version=MODEL_VERSION)
        row["model_correct"] = row["predicted_profitable"] == (row["measured_profitable"] is True)
        if row["model_correct"] != before[key]:
            changed.append({"workload": key[0], "rows": key[1], "cols": key[2],
                            "was_correct": before[key], "now_correct": row["model_correct"]})
    result = Rescore(run=str(bundle.root), device=str(bundle.metadata.get("device", "")),
                     points=len(bundle.summary), correct_before=sum(before.values()),
                     correct_after=sum(r.get("model_correct") is True for r in bundle.summary),
                     changed=tuple(changed))
    if write:
        stamp = datetime.now(timezone.utc).isoformat()
        bundle.save_tables()
        bundle.metadata["cost_model"] = {**bundle.metadata.get("cost_model", {}),
                                         "version": MODEL_VERSION, "rescored_utc": stamp,
                                         "history": HISTORY}
        text, agg = render(bundle.summary, bundle.metadata)
        (bundle.root / "REPORT.md").write_text(text, encoding="utf-8")
        bundle.metadata["report"] = agg
        bundle.save_metadata()
        entry = {"utc": stamp, "model_before": old_version, "model_after": MODEL_VERSION,
                 "points": result.points, "correct_before": result.correct_before,
                 "correct_after": result.correct_after, "changed": list(changed)}
        with (bundle.root / HISTORY).open("a", encoding="utf-8") as fh:
            fh.write(json.dumps(entry) + "\n")
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="re-score split-sweep bundles with the current model")
    ap.add_argument("runs", nargs="+", type=Path)
    ap.add_argument("--write", action="store_true",
                    help="rewrite the bundles and append to their rescore_history.jsonl")
    args = ap.parse_args(argv)
    for run in args.runs:
        r = rescore(run, args.write)
        print(f"{r.run}: {r.correct_before}/{r.points} -> {r.correct_after}/{r.points} "
              f"({len(r.changed)} verdicts changed)")
    if not args.write:
        print("dry run: pass --write to update the bundles")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
