"""Host-side logic of the split sweep: cost-model arithmetic, calibration
text round trip and the summary/model_correct scoring (no GPU)."""
import dataclasses
import math

import pytest

from credit_amd import cost_model
from credit_amd.profile import format_profile_text, make_device_profile, parse_profile_text
from credit_amd.runner import RunConfig, aggregate, build_summary, percentile, summarize
from credit_amd.workloads import WORKLOADS

PARSED = {
    "name": "MI355X", "clock_ghz": 2.4, "cu_count": 256, "xcd_count": 8,
    "lds_bytes_per_cu": 163840, "max_lds_bytes_per_block": 163840, "l2_capacity_bytes": 4194304,
    "l1_latency_cycles": 120.0, "l2_latency_cycles": 285.0, "mall_latency_cycles": 550.0,
    "hbm_latency_cycles": 910.0, "hbm_read_gbps": 6100.0, "hbm_write_gbps": 4600.0,
    "hbm_copy_gbps": 6000.0, "lds_read_bytes_per_cycle_cu": 98.0,
    "lds_write_bytes_per_cycle_cu": 66.0, "exchange_roundtrip_cycles_xcd": 2050.0,
    "exchange_roundtrip_cycles_cross": 2900.0,
}


def test_profile_text_round_trip():
    text = format_profile_text(PARSED)
    back = parse_profile_text(text)
    for k, v in PARSED.items():
        assert back[k] == pytest.approx(v, rel=1e-5) if isinstance(v, float) else back[k] == v


def test_profile_text_missing_key_raises():
    text = format_profile_text(PARSED).replace("HBM read bandwidth", "HBM rd bw")
    with pytest.raises(RuntimeError):
        parse_profile_text(text)


def test_estimate_rejects_bad_inputs():
    prof = make_device_profile(PARSED)
    spec = WORKLOADS["softmax_fwd"]
    with pytest.raises(ValueError):
        cost_model.estimate(spec, 65536, 4, 0.01, prof, baseline_ms=0.0)
    with pytest.raises(ValueError):
        cost_model.estimate(spec, 65536, 1, 0.01, prof, baseline_ms=1.0)


def test_estimate_delta_is_sum_of_terms():
    prof = make_device_profile(PARSED)
    spec = dataclasses.replace(WORKLOADS["softmax_fwd"], rows=512)
    m = cost_model.estimate(spec, 262144, 4, 0.005, prof, baseline_ms=0.3, rows=512)
    assert m.predicted_delta_ms == pytest.approx(
        m.saved_reread_ms + m.fill_gain_ms - m.control_overhead_ms - m.lds_replay_ms
        - m.l2_exchange_ms)
    assert m.predicted_profitable == (m.predicted_delta_ms > 0)


def test_rows_wider_than_staging_save_rereads():
    """A row the STAGED variant cannot hold is re-read by the no-split
    variant; the split saves exactly the re-read share of the baseline."""
    prof = make_device_profile(PARSED)
    spec = dataclasses.replace(WORKLOADS["softmax_fwd"], rows=512)
    m = cost_model.estimate(spec, 262144, 4, 0.0, prof, baseline_ms=0.3, rows=512)
    assert m.saved_reread_ms == pytest.approx(0.3 * 4.0 / 12.0)
    narrow = cost_model.estimate(spec, 4096, 4, 0.0, prof, baseline_ms=0.3, rows=512)
    assert narrow.saved_reread_ms == 0.0


def test_percentile_and_summarize():
    assert percentile([1, 2, 3, 4], 0.5) == pytest.approx(2.5)
    s = summarize([3.0, float("nan"), 1.0, 2.0])
    assert s["median"] == 2.0
    assert math.isnan(summarize([])["median"])


def test_run_config_validation_and_quick():
    with pytest.raises(ValueError):
        RunConfig.from_dict({"workloads": ["ffn"]})
    with pytest.raises(ValueError):
        RunConfig.from_dict({"splits": [1]})
    q = RunConfig.from_dict({"quick": True}).effective()
    assert len(q.n_values) == 2 and q.trials == 1


def _raw(name, rows, cols, block_ms, split_ms):
    out = [{"workload": name, "rows": rows, "cols": cols, "variant": "read", "split": 0,
            "ms": block_ms, "p20_ms": block_ms, "p80_ms": block_ms, "correct": True}]
    for p, ms in split_ms.items():
        out.append({"workload": name, "rows": rows, "cols": cols, "variant": "split", "split": p,
                    "ms": ms, "p20_ms": ms, "p80_ms": ms, "correct": True})
    return out


def test_build_summary_scores_model_like_the_reference():
    """measured_profitable = best split < block; model_correct = agreement
    with the prediction at the best predicted split (runner.py:541-617)."""
    prof = make_device_profile(PARSED)
    cfg = RunConfig()
    raw = _raw("softmax_fwd", 256, 262144, 0.30, {2: 0.35, 4: 0.20}) + \
        _raw("row_sum_max", 16384, 4096, 0.05, {2: 0.06, 4: 0.07})
    control = {(256, 2, 1): 0.004, (256, 4, 1): 0.006, (16384, 2, 1): 0.01, (16384, 4, 1): 0.02}
    summary, sweep = build_summary(raw, control, prof, cfg)
    by = {r["workload"]: r for r in summary}
    assert by["softmax_fwd"]["measured_profitable"] and by["softmax_fwd"]["measured_split"] == 4
    assert not by["row_sum_max"]["measured_profitable"]
    for r in summary:
        assert r["model_correct"] == (r["predicted_profitable"] == r["measured_profitable"])
    assert len(sweep) == 4
    agg = aggregate(summary)
    assert agg["points"] == 2 and 0 <= agg["model_accuracy"] <= 1


def test_write_csv_takes_the_union_of_keys(tmp_path):
    from credit_amd.runner import write_csv

    write_csv(tmp_path / "r.csv", [{"a": 1, "b": 2}, {"a": 3, "error": "x"}])
    lines = (tmp_path / "r.csv").read_text().splitlines()
    assert lines[0] == "a,b,error" and lines[2] == "3,,x"
