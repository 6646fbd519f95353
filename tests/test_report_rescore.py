"""Result bundles: REPORT.md and offline re-scoring (credit_amd.report,
credit_amd.rescore), the roles of dsmem_eval/report.py:29-139 and
scripts/rescore_cost_model.py:99-218.  Host-only: a synthetic bundle is
scored with the nominal MI355X profile."""
import json
from dataclasses import asdict

import pytest

from credit_amd import bundle
from credit_amd import rescore as rs
from credit_amd.cost_model import MI355X_NOMINAL, MODEL_VERSION
from credit_amd.report import render
from credit_amd.runner import RunConfig, build_summary


def synthetic_bundle(tmp_path):
    """Two workloads x two widths; the split is faster only at the wider
    width.  Raw timings, a control table and metadata as the runner writes
    them."""
    raw, control = [], {}
    for name in ("softmax_fwd", "layernorm_backward"):
        for cols, block_ms, split_ms in ((4096, 0.10, 0.13), (262144, 0.40, 0.15)):
            rows = 64
            raw.append(dict(workload=name, rows=rows, cols=cols, variant="read", split=0,
                            ms=block_ms, p20_ms=block_ms, p80_ms=block_ms, correct=True))
            for p in (2, 4):
                raw.append(dict(workload=name, rows=rows, cols=cols, variant="split", split=p,
                                ms=split_ms * (1 + 0.1 * (p == 4)), p20_ms=split_ms,
                                p80_ms=split_ms, correct=True))
                control[(name, cols, p)] = 0.004
    summary, sweep = build_summary(raw, control, MI355X_NOMINAL, RunConfig())
    run = tmp_path / "bundle"
    bundle.write_table(run / "summary.csv", summary, bundle.SUMMARY)
    bundle.write_table(run / "cluster_sweep.csv", sweep, bundle.SWEEP)
    meta = {"device": "test", "arch": "gfx950", "cost_model": {"version": MODEL_VERSION},
            "profile": asdict(MI355X_NOMINAL)}
    (run / "metadata.json").write_text(json.dumps(meta))
    return run, summary, meta


def test_report_grid_and_counts(tmp_path):
    _, summary, meta = synthetic_bundle(tmp_path)
    text, agg = render(summary, meta)
    assert agg["points"] == 4 and agg["split_wins"] == 2
    assert agg["model_correct"] == sum(r["model_correct"] for r in summary)
    assert set(agg["by_workload"]) == {"softmax_fwd", "layernorm_backward"}
    assert len(agg["misses"]) == 4 - agg["model_correct"]
    # one grid row per workload, one column per width
    grid = [l for l in text.splitlines() if l.startswith("| softmax_fwd |")]
    assert len(grid) == 3  # the decision grid row and two rate rows
    assert "| 4096 | 262144 |" in text
    assert "P2 " in grid[0]  # the split (P=2) measured fastest at 262144


def test_rescore_keeps_verdicts_then_repairs_them(tmp_path):
    run, summary, _ = synthetic_bundle(tmp_path)
    correct = sum(bool(r["model_correct"]) for r in summary)
    r = rs.rescore(run)
    assert r.correct_before == r.correct_after == correct and not r.changed
    # Corrupt the stored verdicts; a --write rescore recomputes them and
    # records every change in the bundle's history.
    b = bundle.Bundle.load(run)
    for row in b.summary:
        row["model_correct"] = False
        row["predicted_profitable"] = None
    b.save_tables()
    r = rs.rescore(run, write=True)
    assert r.correct_before == 0 and r.correct_after == correct
    assert len(r.changed) == correct
    history = [json.loads(l) for l in (run / rs.HISTORY).read_text().splitlines()]
    assert history[-1]["correct_after"] == correct and history[-1]["model_after"] == MODEL_VERSION
    meta = json.loads((run / "metadata.json").read_text())
    assert meta["report"]["model_correct"] == correct
    assert f"{correct}/4 points decided correctly" in (run / "REPORT.md").read_text()
    # A second write appends a history line with nothing changed.
    rs.rescore(run, write=True)
    history = [json.loads(l) for l in (run / rs.HISTORY).read_text().splitlines()]
    assert len(history) == 2 and history[-1]["changed"] == []


def test_rescore_rejects_incomplete_bundles(tmp_path):
    run, _, _ = synthetic_bundle(tmp_path)
    (run / "cluster_sweep.csv").unlink()
    with pytest.raises(FileNotFoundError, match="cluster_sweep.csv"):
        rs.rescore(run)
    run2, _, _ = synthetic_bundle(tmp_path / "b2")
    meta = json.loads((run2 / "metadata.json").read_text())
    del meta["profile"]
    (run2 / "metadata.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match="profile"):
        rs.rescore(run2)
