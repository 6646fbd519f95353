"""REPORT.md of a split-sweep bundle.

The reference summarises a run in markdown (dsmem_eval/report.py:29-139).
This report is organised around the two questions the gfx950 sweep answers:

1. Did the cost model pick the right side -- split the row across P
   workgroups or keep it in one -- at each (workload, width) point?  A grid
   of workloads x widths shows the measured winner and whether the model
   agreed, followed by the points it got wrong with both deltas.
2. How close to HBM bandwidth does each side run?  Every point lists the
   no-split and best-split rates as a fraction of the 8 TB/s MI355X peak,
   the rate the roofline of the bench is quoted against.

Rows are the typed summary rows of ``credit_amd.bundle`` (or the dicts
``runner.build_summary`` returns, which carry the same keys and types).
"""
from __future__ import annotations

import math
from collections import defaultdict
from pathlib import Path
from typing import Any

HBM_PEAK_GBPS = 8000.0


def _ok(v: Any) -> bool:
    return v is True


def _num(v: Any) -> float:
    try:
        f = float(v)
    except (TypeError, ValueError):
        return math.nan
    return f


def _cell(row: dict[str, Any]) -> str:
    """Measured winner at a point and the model's verdict on it."""
    winner = f"P{row['measured_split']}" if _ok(row.get("measured_profitable")) else "one WG"
    return f"{winner} {'ok' if _ok(row.get('model_correct')) else 'MISS'}"


def summarize(rows: list[dict[str, Any]]) -> dict[str, Any]:
    """Counts behind the report: overall and per workload."""
    scored = [r for r in rows if r.get("model_correct") is not None]
    per: dict[str, dict[str, int]] = defaultdict(lambda: {"points": 0, "split_wins": 0,
                                                          "model_correct": 0})
    for r in scored:
        p = per[str(r["workload"])]
        p["points"] += 1
        p["split_wins"] += _ok(r.get("measured_profitable"))
        p["model_correct"] += _ok(r.get("model_correct"))
    misses = [{"workload": r["workload"], "cols": int(r["cols"]), "rows": int(r["rows"]),
               "measured_delta_ms": _num(r.get("block_ms")) - _num(r.get("split_ms")),
               "predicted_delta_ms": _num(r.get("predicted_delta_ms"))}
              for r in scored if not _ok(r.get("model_correct"))]
    correct = sum(p["model_correct"] for p in per.values())
    return {
        "points": len(scored),
        "model_correct": correct,
        "accuracy": correct / len(scored) if scored else math.nan,
        "split_wins": sum(p["split_wins"] for p in per.values()),
        "by_workload": dict(sorted(per.items())),
        "misses": misses,
    }


def render(rows: list[dict[str, Any]], metadata: dict[str, Any]) -> tuple[str, dict[str, Any]]:
    """(markdown, aggregate) for a bundle's summary rows and metadata."""
    agg = summarize(rows)
    agg["device"] = str(metadata.get("device", ""))
    model = metadata.get("cost_model", {}).get("version", "unknown model")
    device = f"{metadata.get('device', 'unknown device')} ({metadata.get('arch', '?')})"
    acc = agg["accuracy"]
    out = [f"# Split-row sweep on {device}", "",
           f"Cost model `{model}`: {agg['model_correct']}/{agg['points']} points decided "
           f"correctly ({100 * acc:.1f}%)." if agg["points"] else "No scored points.",
           f"Splitting the row measured faster at {agg['split_wins']} of them.", "",
           "## Decisions by workload and width", "",
           "Each cell: the measured winner (`P<k>`: split over k workgroups; `one WG`: the "
           "best single-workgroup variant) and whether the model chose the same side.", ""]
    widths = sorted({int(r["cols"]) for r in rows})
    by_point = {(str(r["workload"]), int(r["cols"])): r for r in rows}
    names = sorted({str(r["workload"]) for r in rows})
    out.append("| workload | " + " | ".join(str(w) for w in widths) + " | correct |")
    out.append("|---|" + "---|" * len(widths) + "---:|")
    for name in names:
        cells = [(_cell(by_point[(name, w)]) if (name, w) in by_point else "") for w in widths]
        p = agg["by_workload"].get(name, {"points": 0, "model_correct": 0})
        out.append(f"| {name} | " + " | ".join(cells) +
                   f" | {p['model_correct']}/{p['points']} |")
    out += ["", "## Points the model got wrong", ""]
    if agg["misses"]:
        out += ["| workload | rows | cols | measured gain of the split (ms) | predicted (ms) |",
                "|---|---:|---:|---:|---:|"]
        for m in agg["misses"]:
            out.append(f"| {m['workload']} | {m['rows']} | {m['cols']} | "
                       f"{m['measured_delta_ms']:+.4f} | {m['predicted_delta_ms']:+.4f} |")
    else:
        out.append("None.")
    out += ["", "## HBM rate of each side", "",
            f"Algorithmic bytes over the median time, and its fraction of {HBM_PEAK_GBPS:.0f} GB/s.",
            "", "| workload | rows | cols | one-WG variant | one WG GB/s | frac | best P | "
            "split GB/s | frac | predicted P |", "|---|---:|---:|---|---:|---:|---:|---:|---:|---:|"]
    for r in sorted(rows, key=lambda r: (str(r["workload"]), int(r["cols"]))):
        bg, sg = _num(r.get("block_gbps")), _num(r.get("split_gbps"))
        out.append(f"| {r['workload']} | {int(r['rows'])} | {int(r['cols'])} | "
                   f"{r.get('block_variant', '')} | {bg:.0f} | {bg / HBM_PEAK_GBPS:.3f} | "
                   f"{r.get('measured_split', '')} | {sg:.0f} | {sg / HBM_PEAK_GBPS:.3f} | "
                   f"{r.get('predicted_split', '')} |")
    return "\n".join(out) + "\n", agg


def write_report(output_dir: Path, rows: list[dict[str, Any]],
                 metadata: dict[str, Any]) -> dict[str, Any]:
    text, agg = render(rows, metadata)
    (Path(output_dir) / "REPORT.md").write_text(text, encoding="utf-8")
    return agg
