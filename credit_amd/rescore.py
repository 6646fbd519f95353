"""Re-score saved result bundles with the current cost model (the role of
scripts/rescore_cost_model.py:99-218).

    python -m credit_amd.rescore RUN_DIR [RUN_DIR ...] [--write]

For every cluster_sweep.csv row the prediction is recomputed from the
bundle's own measurements -- the calibrated device profile in metadata.json,
the row's measured control overhead and the point's best no-split time --
so a bundle measured once on an MI355X can be re-scored after a model change
without the GPU.  A dry run prints old -> new correct counts; --write keeps
the first pre-rescore copies as summary.prev_model.csv /
cluster_sweep.prev_model.csv, rewrites both CSVs, REPORT.md and the
metadata's cost_model and aggregate fields.  Host-only: no GPU is touched.
"""
from __future__ import annotations

import argparse
import csv
import dataclasses
import json
import shutil
from collections import defaultdict
from pathlib import Path
from typing import Any

from .cost_model import MODEL_VERSION, DeviceProfile, estimate
from .report import build_report, truth
from .workloads import WORKLOADS


def read_csv(path: Path) -> list[dict[str, str]]:
    with path.open(newline="", encoding="utf-8") as fh:
        return list(csv.DictReader(fh))


def write_csv(path: Path, rows: list[dict[str, Any]]) -> None:
    if not rows:
        return
    fields: list[str] = []
    for r in rows:
        fields += [k for k in r if k not in fields]
    tmp = path.with_suffix(path.suffix + ".tmp")
    with tmp.open("w", newline="", encoding="utf-8") as fh:
        w = csv.DictWriter(fh, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)
    tmp.replace(path)


def profile_from_metadata(metadata: dict[str, Any]) -> DeviceProfile:
    """The calibrated profile the runner stored (profile_as_dict)."""
    raw = metadata.get("profile")
    if not raw:
        raise ValueError("metadata.json has no calibrated 'profile' (an incomplete run?)")
    kinds = {f.name: f.type for f in dataclasses.fields(DeviceProfile)}
    missing = sorted(set(kinds) - set(raw))
    if missing:
        raise ValueError(f"metadata profile lacks {missing}")
    conv = {"str": str, "int": int, "float": float}
    return DeviceProfile(**{k: conv[t if isinstance(t, str) else t.__name__](raw[k])
                            for k, t in kinds.items()})


def rescore(run: Path, write: bool = False) -> dict[str, Any]:
    run = Path(run).resolve()
    paths = {n: run / n for n in ("summary.csv", "cluster_sweep.csv", "metadata.json")}
    missing = [n for n, p in paths.items() if not p.exists()]
    if missing:
        raise FileNotFoundError(f"{run}: missing {', '.join(missing)}")
    metadata = json.loads(paths["metadata.json"].read_text(encoding="utf-8"))
    profile = profile_from_metadata(metadata)
    summary: list[dict[str, Any]] = read_csv(paths["summary.csv"])
    sweep: list[dict[str, Any]] = read_csv(paths["cluster_sweep.csv"])
    point = {(r["workload"], int(r["rows"]), int(r["cols"])): r for r in summary}
    old_correct = sum(truth(r.get("model_correct")) for r in summary)

    estimates: dict[tuple[str, int, int], list[tuple[float, int, bool]]] = defaultdict(list)
    for r in sweep:
        key = (r["workload"], int(r["rows"]), int(r["cols"]))
        if key not in point:
            continue
        spec = dataclasses.replace(WORKLOADS[r["workload"]], rows=key[1])
        m = estimate(spec, key[2], int(r["split"]), float(r["control_overhead_ms"]), profile,
                     baseline_ms=float(point[key]["block_ms"]), rows=key[1])
        r.update({"model_version": MODEL_VERSION, **dataclasses.asdict(m)})
        estimates[key].append((m.predicted_delta_ms, int(r["split"]), m.predicted_profitable))

    for key, r in point.items():
        if not estimates[key]:
            continue
        delta, split, profitable = max(estimates[key], key=lambda e: e[0])
        measured = truth(r["measured_profitable"])
        r.update({"model_version": MODEL_VERSION, "predicted_split": split,
                  "predicted_delta_ms": delta, "predicted_profitable": profitable,
                  "model_correct": profitable == measured})
    new_correct = sum(truth(r.get("model_correct")) for r in summary)
    result = {"run": str(run), "device": str(metadata.get("device", "")),
              "points": len(summary), "old_correct": old_correct, "new_correct": new_correct}
    if not write:
        return result
    for name in ("summary.csv", "cluster_sweep.csv"):
        backup = run / name.replace(".csv", ".prev_model.csv")
        if not backup.exists():
            shutil.copy2(paths[name], backup)
    write_csv(paths["summary.csv"], summary)
    write_csv(paths["cluster_sweep.csv"], sweep)
    report, aggregate = build_report(summary, metadata)
    (run / "REPORT.md").write_text(report, encoding="utf-8")
    metadata["cost_model"] = {**metadata.get("cost_model", {}), "version": MODEL_VERSION,
                              "previous_correct": old_correct, "revised_correct": new_correct,
                              "points": len(summary)}
    metadata["report"] = aggregate
    paths["metadata.json"].write_text(json.dumps(metadata, indent=2) + "\n", encoding="utf-8")
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("runs", nargs="+", type=Path)
    ap.add_argument("--write", action="store_true",
                    help="rewrite the bundles (first copies kept as *.prev_model.csv)")
    args = ap.parse_args(argv)
    for run in args.runs:
        r = rescore(run, args.write)
        print(f"{r['run']}: {r['old_correct']}/{r['points']} -> {r['new_correct']}/{r['points']}")
    if not args.write:
        print("Dry run; pass --write to update the bundles.")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
