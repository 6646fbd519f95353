"""Host-side logic of the split sweep: cost-model arithmetic, calibration
text round trip and the summary/model_correct scoring (no GPU)."""
import dataclasses
import math

import pytest

from credit_amd import cost_model
from credit_amd.profile import format_profile_text, make_device_profile, parse_profile_text
from credit_amd.runner import RunConfig, aggregate, build_summary
from credit_amd.timing import TrialStats
from credit_amd.workloads import WORKLOADS

PARSED = {
    "name": "MI355X", "clock_ghz": 2.4, "cu_count": 256, "xcd_count": 8,
    "lds_bytes_per_cu": 163840, "max_lds_bytes_per_block": 163840, "l2_capacity_bytes": 4194304,
    "l1_latency_cycles": 120.0, "l2_latency_cycles": 285.0, "mall_latency_cycles": 550.0,
    "hbm_latency_cycles": 910.0, "hbm_read_gbps": 6100.0, "hbm_write_gbps": 4600.0,
    "hbm_copy_gbps": 6000.0, "lds_read_bytes_per_cycle_cu": 98.0,
    "lds_write_bytes_per_cycle_cu": 66.0, "exchange_roundtrip_cycles_xcd": 2050.0,
    "exchange_roundtrip_cycles_cross": 2900.0, "l1_read_bytes_per_cycle_cu": 64.0,
    "l2_read_bytes_per_cycle_xcd": 1024.0, "l2_read_gbps": 19000.0,
    "slot_store_bytes_per_cycle_wg": 2.5, "slot_store_gbps": 1500.0,
    "ticket_cycles_private": 900.0, "ticket_cycles_shared": 4000.0,
    "mfma_bf16_tflops": 2300.0, "mfma_clock_mhz": 2250.0,
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
        - m.l2_exchange_ms + m.hidden_sync_ms)
    assert m.predicted_profitable == (m.predicted_delta_ms > 0)


def test_pipelined_split_hides_at_most_depth_stream_steps_of_sync():
    """The group pipelines hide control + exchange up to DEPTH times the
    compulsory stream time (the softmax forward's parked 512-lane shape at
    C4: 16 members of 4096 vectors, DEPTH 4); a barrier-synchronised slice
    kernel (depth 0) hides none.  A control overhead beyond that is charged."""
    prof = make_device_profile(PARSED)
    piped = dataclasses.replace(WORKLOADS["softmax_fwd"], rows=512)
    flat = dataclasses.replace(piped, split_pipeline_depth=0)
    assert piped.split_pipeline_depth(262144, 16) == 4
    for ctl in (0.001, 0.05, 5.0):
        a = cost_model.estimate(piped, 262144, 16, ctl, prof, baseline_ms=0.3, rows=512)
        b = cost_model.estimate(flat, 262144, 16, ctl, prof, baseline_ms=0.3, rows=512)
        sync = a.control_overhead_ms + a.l2_exchange_ms
        remaining = 0.3 - a.saved_reread_ms
        assert b.hidden_sync_ms == 0.0
        assert a.hidden_sync_ms == pytest.approx(min(sync, 4 * remaining))
        assert a.predicted_delta_ms - b.predicted_delta_ms == pytest.approx(a.hidden_sync_ms)
    assert cost_model.estimate(piped, 262144, 16, 5.0, prof, baseline_ms=0.3,
                               rows=512).predicted_profitable is False


@pytest.mark.parametrize("name,cols,split,depth", [
    ("rmsnorm_fwd", 131072, 8, 4),             # 2048 vectors per member: group pipeline
    ("rmsnorm_fwd", 131072, 2, 0),             # 8192: slice kernel
    ("rmsnorm_fwd", 131072, 16, 0),            # 1024: slice kernel
    ("rmsnorm_fwd", 65544, 5, 4),              # 1639 (the last member 1637)
    ("layernorm_backward_bf16", 65536, 8, 4),  # 1024 vectors, 8 members
    ("layernorm_backward_bf16", 65536, 2, 0),  # 4096 vectors: slice kernel
    ("layernorm_backward_bf16", 262144, 32, 0),  # more than 16 members
    ("softmax_fwd", 262144, 16, 4),            # 4096 f32x4: the parked shape
    ("softmax_fwd", 262144, 32, 2),
    ("softmax_bwd", 262144, 32, 4),            # 2048 f32x4: the parked shape
    ("softmax_bwd", 262144, 64, 2),
    ("rmsnorm_bwd", 131072, 16, 4),
    ("row_sum_max", 65536, 4, 0),
])
def test_pipeline_depth_follows_the_kernel_each_split_runs(name, cols, split, depth):
    d = WORKLOADS[name].split_pipeline_depth
    assert (d(cols, split) if callable(d) else d) == depth


def test_rows_wider_than_staging_save_rereads():
    """A row the STAGED variant cannot hold is re-read by the no-split
    variant; the split saves exactly the re-read share of the baseline."""
    prof = make_device_profile(PARSED)
    spec = dataclasses.replace(WORKLOADS["softmax_fwd"], rows=512)
    m = cost_model.estimate(spec, 262144, 4, 0.0, prof, baseline_ms=0.3, rows=512)
    assert m.saved_reread_ms == pytest.approx(0.3 * 4.0 / 12.0)
    narrow = cost_model.estimate(spec, 4096, 4, 0.0, prof, baseline_ms=0.3, rows=512)
    assert narrow.saved_reread_ms == 0.0


def test_trial_stats_quantiles():
    """Median and inclusive-method 20th/80th percentiles: with samples
    1..5 the percentiles sit at 0.8 and 3.2 positions of the sorted list."""
    t = TrialStats((5.0, 1.0, 3.0, 2.0, 4.0), iters=20)
    assert t.median_ms == 3.0
    assert t.p20_ms == pytest.approx(1.8) and t.p80_ms == pytest.approx(4.2)
    assert t.as_dict()["trials"] == 5 and t.as_dict()["iters"] == 20
    one = TrialStats((2.5,), iters=20)
    assert one.median_ms == one.p20_ms == one.p80_ms == 2.5
    nan = TrialStats((float("nan"), 1.0, 3.0), iters=1)
    assert nan.median_ms == 2.0
    assert math.isnan(TrialStats((), iters=1).median_ms)


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
    control = {("softmax_fwd", 262144, 2): 0.004, ("softmax_fwd", 262144, 4): 0.006,
               ("row_sum_max", 4096, 2): 0.01, ("row_sum_max", 4096, 4): 0.02}
    summary, sweep = build_summary(raw, control, prof, cfg)
    by = {r["workload"]: r for r in summary}
    assert by["softmax_fwd"]["measured_profitable"] and by["softmax_fwd"]["measured_split"] == 4
    assert not by["row_sum_max"]["measured_profitable"]
    for r in summary:
        assert r["model_correct"] == (r["predicted_profitable"] == r["measured_profitable"])
    assert len(sweep) == 4
    agg = aggregate(summary)
    assert agg["points"] == 2 and 0 <= agg["model_accuracy"] <= 1


def test_bundle_tables_round_trip_typed(tmp_path):
    """Tables are written in schema order and read back with their types;
    a missing value reads as None, NaN survives, an unknown column is an
    error on write."""
    from credit_amd import bundle

    rows = [{"workload": "softmax_fwd", "rows": 512, "cols": 262144, "variant": "split",
             "split": 4, "correct": True, "ms": 0.25, "p20_ms": 0.24, "p80_ms": 0.26,
             "samples": 5},
            {"workload": "softmax_fwd", "rows": 512, "cols": 262144, "variant": "split",
             "split": 64, "ms": float("nan"), "error": "-4: unsupported"}]
    path = tmp_path / "raw.csv"
    bundle.write_table(path, rows, bundle.RAW)
    assert path.read_text().splitlines()[0] == ",".join(n for n, _ in bundle.RAW)
    back = bundle.read_table(path, bundle.RAW)
    assert back[0]["correct"] is True and back[0]["split"] == 4 and back[0]["ms"] == 0.25
    assert back[1]["correct"] is None and math.isnan(back[1]["ms"])
    assert back[1]["error"] == "-4: unsupported"
    with pytest.raises(ValueError):
        bundle.write_table(path, [{"workload": "x", "surprise": 1}], bundle.RAW)
