"""REPORT.md of a result bundle (the role of dsmem_eval/report.py:29-139).

A bundle is the directory the runner writes (credit_amd.runner.run_suite):
metadata.json, summary.csv (one row per workload x width: best no-split
variant, best split, the cost model's prediction), cluster_sweep.csv (one
row per split factor), raw.csv, control.csv.  The report states how often
splitting a row across workgroups beat the best single-workgroup variant,
how often the cost model predicted that sign correctly, the results at the
widest swept row, and where each workload's split first pays off (measured
and predicted).  Rows read back from CSV carry strings; every field is
converted here.
"""
from __future__ import annotations

import math
from collections import defaultdict
from pathlib import Path
from typing import Any, Iterable


def truth(value: Any) -> bool:
    if isinstance(value, bool):
        return value
    return str(value).strip().lower() == "true"


def _finite(value: Any) -> bool:
    try:
        return math.isfinite(float(value))
    except (TypeError, ValueError):
        return False


def geometric_mean(values: Iterable[float]) -> float:
    positive = [v for v in values if v > 0.0 and math.isfinite(v)]
    if not positive:
        return math.nan
    return math.exp(sum(math.log(v) for v in positive) / len(positive))


def crossovers(summary_rows: list[dict[str, Any]]) -> list[dict[str, Any]]:
    """Per workload, the narrowest swept width at which the split measured
    (and was predicted) faster than the best no-split variant; None when it
    never was."""
    by_workload: dict[str, list[dict[str, Any]]] = defaultdict(list)
    for row in summary_rows:
        by_workload[str(row["workload"])].append(row)
    out = []
    for name, rows in sorted(by_workload.items()):
        ordered = sorted(rows, key=lambda r: int(r["cols"]))
        measured = next((int(r["cols"]) for r in ordered if truth(r.get("measured_profitable"))), None)
        predicted = next((int(r["cols"]) for r in ordered if truth(r.get("predicted_profitable"))),
                         None)
        out.append({"workload": name, "label": str(ordered[0].get("label", name)),
                    "predicted": predicted, "measured": measured})
    return out


def build_report(summary_rows: list[dict[str, Any]],
                 metadata: dict[str, Any]) -> tuple[str, dict[str, Any]]:
    """(markdown, aggregate) for a bundle's summary rows and metadata."""
    valid = [r for r in summary_rows if _finite(r.get("split_vs_block"))]
    wins = sum(float(r["split_vs_block"]) > 1.0 for r in valid)
    model_rows = [r for r in summary_rows if "model_correct" in r]
    model_correct = sum(truth(r["model_correct"]) for r in model_rows)
    widest = max((int(r["cols"]) for r in valid), default=0)
    widest_rows = sorted((r for r in valid if int(r["cols"]) == widest),
                         key=lambda r: str(r["workload"]))
    widest_geomean = geometric_mean(float(r["split_vs_block"]) for r in widest_rows)
    version = metadata.get("cost_model", {}).get("version", "")
    device = f"{metadata.get('device', 'unknown device')} ({metadata.get('arch', '')})"
    lines = [
        f"# Split-row evaluation on {device}",
        "",
        f"- Splitting a row across workgroups beats the best single-workgroup variant on "
        f"{wins}/{len(valid)} workload-width points.",
        f"- The cost model ({version}) predicts {model_correct}/{len(model_rows)} "
        f"profitability signs correctly.",
    ]
    if widest:
        lines.append(f"- At N={widest}, the best split is {widest_geomean:.3f}x the best "
                     f"single-workgroup variant (geometric mean over workloads).")
    lines += ["", f"## Results at N={widest}", "",
              "| Workload | rows | no-split | no-split ms | split ms | split / no-split | P | "
              "predicted P | model correct |",
              "|---|---:|---|---:|---:|---:|---:|---:|---|"]
    for r in widest_rows:
        lines.append(
            f"| {r.get('label', r['workload'])} | {int(r['rows'])} | {r['block_variant']} "
            f"| {float(r['block_ms']):.4f} | {float(r['split_ms']):.4f} "
            f"| {float(r['split_vs_block']):.3f}x | {int(float(r['measured_split']))} "
            f"| {int(float(r['predicted_split']))} | {truth(r.get('model_correct'))} |")
    cross = crossovers(summary_rows)
    lines += ["", "## Crossover validation", "",
              "Narrowest swept width at which the split is faster than the best "
              "single-workgroup variant.", "",
              "| Workload | Predicted | Measured |", "|---|---:|---:|"]
    for c in cross:
        pred = "none" if c["predicted"] is None else str(c["predicted"])
        meas = "none" if c["measured"] is None else str(c["measured"])
        lines.append(f"| {c['label']} | {pred} | {meas} |")
    lines += ["", "## All points", "",
              "| workload | rows | cols | no-split | no-split ms | split ms | best P | "
              "no-split GB/s | split GB/s | predicted | measured | correct |",
              "|---|---:|---:|---|---:|---:|---:|---:|---:|---|---|---|"]
    for r in sorted(valid, key=lambda r: (str(r["workload"]), int(r["cols"]))):
        lines.append(
            f"| {r['workload']} | {int(r['rows'])} | {int(r['cols'])} | {r['block_variant']} "
            f"| {float(r['block_ms']):.4f} | {float(r['split_ms']):.4f} "
            f"| {int(float(r['measured_split']))} | {float(r['block_gbps']):.0f} "
            f"| {float(r['split_gbps']):.0f} | {truth(r.get('predicted_profitable'))} "
            f"| {truth(r.get('measured_profitable'))} | {truth(r.get('model_correct'))} |")
    aggregate = {
        "device": str(metadata.get("device", "")),
        "points": len(valid),
        "split_wins": wins,
        "model_points": len(model_rows),
        "model_correct": model_correct,
        "largest_width": widest,
        "largest_width_geomean_speedup": widest_geomean,
        "crossovers": cross,
    }
    return "\n".join(lines) + "\n", aggregate


def write_report(output_dir: Path, summary_rows: list[dict[str, Any]],
                 metadata: dict[str, Any]) -> dict[str, Any]:
    report, aggregate = build_report(summary_rows, metadata)
    (Path(output_dir) / "REPORT.md").write_text(report, encoding="utf-8")
    return aggregate
