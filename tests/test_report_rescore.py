"""Result bundles: REPORT.md and offline re-scoring (credit_amd.report,
credit_amd.rescore), the roles of dsmem_eval/report.py:29-139 and
scripts/rescore_cost_model.py:99-218.  Host-only: a synthetic bundle is
scored with the nominal MI355X profile."""
import csv
import json
from dataclasses import asdict

from credit_amd import rescore as rs
from credit_amd.cost_model import MI355X_NOMINAL, MODEL_VERSION
from credit_amd.report import build_report
from credit_amd.runner import RunConfig, build_summary, write_csv


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
                for barriers in (1, 2):
                    control[(rows, p, barriers)] = 0.004
    summary, sweep = build_summary(raw, control, MI355X_NOMINAL, RunConfig())
    run = tmp_path / "bundle"
    write_csv(run / "summary.csv", summary)
    write_csv(run / "cluster_sweep.csv", sweep)
    meta = {"device": "test", "arch": "gfx950", "cost_model": {"version": MODEL_VERSION},
            "profile": asdict(MI355X_NOMINAL)}
    (run / "metadata.json").write_text(json.dumps(meta))
    return run, summary, meta


def test_report_counts_and_crossovers(tmp_path):
    _, summary, meta = synthetic_bundle(tmp_path)
    text, agg = build_report(summary, meta)
    assert agg["points"] == 4 and agg["split_wins"] == 2
    assert agg["largest_width"] == 262144
    assert abs(agg["largest_width_geomean_speedup"] - 0.40 / 0.15) < 1e-9
    cross = {c["workload"]: c for c in agg["crossovers"]}
    assert cross["softmax_fwd"]["measured"] == 262144
    assert "## All points" in text and text.count("| softmax_fwd |") == 2


def test_rescore_reproduces_then_repairs(tmp_path):
    run, summary, _ = synthetic_bundle(tmp_path)
    correct = sum(bool(r["model_correct"]) for r in summary)
    r = rs.rescore(run)
    assert r["old_correct"] == r["new_correct"] == correct  # same model, same verdicts
    # Corrupt the stored verdicts; a --write rescore recomputes them.
    path = run / "summary.csv"
    rows = list(csv.DictReader(path.open()))
    for row in rows:
        row["model_correct"] = "False"
        row["predicted_profitable"] = "garbage"
    rs.write_csv(path, rows)
    r = rs.rescore(run, write=True)
    assert r["old_correct"] == 0 and r["new_correct"] == correct
    assert (run / "summary.prev_model.csv").exists() and (run / "REPORT.md").exists()
    meta = json.loads((run / "metadata.json").read_text())
    assert meta["cost_model"]["revised_correct"] == correct
    assert f"predicts {correct}/4" in (run / "REPORT.md").read_text()
    # A second --write keeps the first backup.
    first = (run / "summary.prev_model.csv").read_text()
    rs.rescore(run, write=True)
    assert (run / "summary.prev_model.csv").read_text() == first


def test_rescore_rejects_incomplete_bundles(tmp_path):
    run, _, _ = synthetic_bundle(tmp_path)
    (run / "cluster_sweep.csv").unlink()
    try:
        rs.rescore(run)
    except FileNotFoundError as err:
        assert "cluster_sweep.csv" in str(err)
    else:
        raise AssertionError("missing file accepted")
