"""Host logic of the split-sweep counter pass (no GPU): the plan names the
timed sweep's rows, dispatches are attributed to entries by their marker,
and the merged columns land beside the cost model's predicted traffic."""
import csv
import dataclasses
import math

import pytest

from credit_amd import bundle, counters
from credit_amd.cost_model import MI355X_NOMINAL, predict_traffic
from credit_amd.runner import sweep_rows, variant_list
from credit_amd.workloads import WORKLOADS

HEADER = ["Correlation_Id", "Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name",
          "Counter_Value"]
MARK = "void credit::(anonymous namespace)::transpose_bf16_kernel(unsigned short const*, int)"
KERN = "void credit::(anonymous namespace)::softmax_fwd_group_kernel<512, 8>(float const*)"
FILL = "void credit::(anonymous namespace)::fill_u32_kernel(unsigned int*, unsigned int, long)"


def _csv(path, counter, dispatches):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(HEADER)
        for i, (name, grid, value) in enumerate(dispatches, start=1):
            w.writerow([i, i, grid, name, counter, value])


def test_plan_matches_the_sweep_rows_and_variants():
    plan = counters.build_plan(("softmax_fwd", "rmsnorm_bwd"), (4096, 262144), (2, 8), 64 << 20)
    assert [e["index"] for e in plan] == list(range(len(plan)))
    for name in ("softmax_fwd", "rmsnorm_bwd"):
        spec = WORKLOADS[name]
        for cols in (4096, 262144):
            got = [(e["variant"], e["split"]) for e in plan
                   if e["workload"] == name and e["cols"] == cols]
            assert got == variant_list(spec, cols, (2, 8))
            assert {e["rows"] for e in plan if e["workload"] == name and e["cols"] == cols} == \
                {sweep_rows(spec, cols, 64 << 20)}


def test_dispatches_are_summed_per_marker(tmp_path):
    """Entry i's marker has i + 2 workgroups; a one-workgroup marker closes
    the previous entry (input preparation of the next point belongs to no
    entry), and a call's every kernel counts."""
    p = tmp_path / "f.csv"
    _csv(p, "FETCH_SIZE", [
        (FILL, 256, 99.0),          # before any marker: ignored
        (MARK, 2 * 256, 1.0),       # entry 0
        (KERN, 131072, 10.0), (FILL, 256, 2.0),
        (MARK, 256, 1.0),           # idle: the next point's input preparation
        (FILL, 4096, 50.0),
        (MARK, 3 * 256, 1.0),       # entry 1
        (KERN, 131072, 7.0),
    ])
    sums = counters.entry_sums(p)
    assert sums[0]["FETCH_SIZE"] == 12.0
    assert sums[1]["FETCH_SIZE"] == 7.0
    assert set(sums) == {0, 1}


def test_predicted_traffic_terms():
    """One HBM pass plus the slot traffic for the split, the re-read for a no-split variant whose
    row does not fit, none where it fits; L2 requests count 128-byte read
    lines and 64-byte write requests (softmax forward: 1:1, so 1.5x the
    line count) plus the exchange's slot stores and polls."""
    spec = dataclasses.replace(WORKLOADS["softmax_fwd"], rows=256)
    wide = predict_traffic(spec, 262144, 16, MI355X_NOMINAL, rows=256)
    compulsory = spec.algorithmic_bytes(256, 262144)
    assert wide.hbm_bytes == compulsory + wide.exchange_bytes
    assert wide.block_hbm_bytes == pytest.approx(compulsory + 256 * 262144 *
                                                 spec.reread_bytes_per_element)
    narrow = predict_traffic(spec, 4096, 2, MI355X_NOMINAL, rows=256)
    assert narrow.block_hbm_bytes == spec.algorithmic_bytes(256, 4096)
    stream = 1.5 * compulsory / 128
    assert stream < wide.l2_requests < stream * 1.01
    # 256 rows x one stage x 16 members, two partials (max, sum): two slot
    # stores + ceil(2 * 16 * 8 / 128) poll lines each
    assert spec.partial_count == 2 and spec.barrier_count == 1
    assert wide.l2_requests - stream == pytest.approx(256 * 16 * (2 + 2), rel=1e-9, abs=1e-3)
    assert wide.exchange_bytes == 256 * 16 * (2 * 8 + 2 * 8 * 16)
    assert wide.lds_bytes > 0


def test_merge_fills_the_sweep_beside_predictions(tmp_path):
    """A two-entry plan (read, split 2) at one point: the split row gets
    measured bytes = FETCH x fetch scale + WRITE x write scale, the block
    variant's bytes beside them, and the L2 request count."""
    import json

    b = tmp_path / "bundle"
    b.mkdir()
    summary = [{"workload": "softmax_fwd", "rows": 8, "cols": 4096, "block_variant": "read"}]
    sweep = [{"workload": "softmax_fwd", "rows": 8, "cols": 4096, "split": 2,
              "predicted_hbm_bytes": 300000.0, "predicted_block_hbm_bytes": 280000.0,
              "predicted_l2_requests": 2000.0}]
    bundle.write_table(b / "summary.csv", summary, bundle.SUMMARY)
    bundle.write_table(b / "cluster_sweep.csv", sweep, bundle.SWEEP)
    bundle.write_table(b / "raw.csv", [], bundle.RAW)
    (b / "metadata.json").write_text("{}\n")
    plan = {"entries": [{"index": 0, "workload": "softmax_fwd", "rows": 8, "cols": 4096,
                         "variant": "read", "split": 0, "status": "ok"},
                        {"index": 1, "workload": "softmax_fwd", "rows": 8, "cols": 4096,
                         "variant": "split", "split": 2, "status": "ok"}]}
    (tmp_path / "plan.json").write_text(json.dumps(plan))
    copy = "void credit::(anonymous namespace)::mb_stream_kernel<1, 1, 4, 1>(StreamArgs)"
    _csv(tmp_path / "cf.csv", "FETCH_SIZE", [(copy, 256, 512.0)])   # 1 MiB copy: x2048/KiB
    _csv(tmp_path / "cw.csv", "WRITE_SIZE", [(copy, 256, 1024.0)])  # x1024/KiB
    _csv(tmp_path / "f.csv", "FETCH_SIZE", [(MARK, 512, 0), (KERN, 4096, 100.0),
                                            (MARK, 768, 0), (KERN, 4096, 110.0)])
    _csv(tmp_path / "w.csv", "WRITE_SIZE", [(MARK, 512, 0), (KERN, 4096, 50.0),
                                            (MARK, 768, 0), (KERN, 4096, 60.0)])
    _csv(tmp_path / "t.csv", "TCC_REQ_sum", [(MARK, 512, 0), (KERN, 4096, 1800.0),
                                             (MARK, 768, 0), (KERN, 4096, 2100.0)])
    # Two kernels in the split call: the LDS instruction count is their sum.
    _csv(tmp_path / "l.csv", "SQ_INSTS_LDS", [(MARK, 512, 0), (KERN, 4096, 70.0),
                                              (MARK, 768, 0), (KERN, 4096, 300.0),
                                              (KERN, 4096, 20.0)])
    res = counters.merge(b, tmp_path / "plan.json", tmp_path / "f.csv", tmp_path / "w.csv",
                         tmp_path / "cf.csv", tmp_path / "cw.csv", 1 << 20, tmp_path / "t.csv",
                         tmp_path / "l.csv")
    assert res["sweep_rows_filled"] == 1
    row = bundle.read_table(b / "cluster_sweep.csv", bundle.SWEEP)[0]
    assert row["measured_hbm_bytes"] == pytest.approx(110.0 * 2048 + 60.0 * 1024)
    assert row["measured_block_hbm_bytes"] == pytest.approx(100.0 * 2048 + 50.0 * 1024)
    assert row["measured_l2_requests"] == 2100.0
    assert row["measured_lds_instructions"] == 320.0
    ratios = counters.agreement(b)
    assert len(ratios) == 1 and math.isfinite(ratios[0]["hbm_ratio"])
    # per row (8) and member (2)
    assert ratios[0]["lds_insts_per_row_member"] == pytest.approx(320.0 / 16)
    assert "SQ_INSTS_LDS" in counters.traffic_report(b)
