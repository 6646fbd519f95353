"""bench.py's printed line, host side (no GPU): the --gpus guard, the
compact suite entries (the whole line must fit the ~8.5 KB of stdout a
driver keeps, with every C1-C5 workload in it) and the rule that a PMC
traffic figure is reported only while its kernel sources hash as they did
when the counters were taken."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from credit_amd import hip_lib  # noqa: E402
from credit_amd.traffic import source_fingerprints  # noqa: E402

C1_C5 = ("row_sum_max", "layernorm_fwd", "rmsnorm_fwd", "rmsnorm_bwd", "rmsnorm_fwd_bwd",
         "softmax_fwd", "softmax_bwd", "ffn")


def test_more_than_one_gpu_is_refused_before_any_gpu_work():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert out.returncode == 2
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def synthetic_entry(name, ffn):
    """A measure() record with the fields compact() reads, sized like a real one
    (the variant sweep and trial lists it drops included)."""
    ceiling = ({"TFLOPs": 2431.28, "frac": 0.5856} if ffn else
               {"mix": "2:1", "GBps": 6393.4, "ms": 0.25, "frac": 0.8939,
                "shape": {"lanes": 64, "vectors_per_lane": 4, "workgroups_per_cu": 4,
                          "nontemporal_stores": True}, "bytes": 1610612736})
    roof = {"bound": "mfma" if ffn else "hbm", "achieved": 1422.84 if ffn else 5715.2,
            "peak": 2500.0 if ffn else 8000.0, "unit": "TFLOP/s" if ffn else "GB/s",
            "frac": 0.5691, "frac_median": 0.5678, "traffic": None if ffn else 1613000000,
            "traffic_source": "PMC at 0123456789ab", "ceiling": ceiling}
    return {"rows": 4096, "cols": 65536, "ms_per_step": 0.282, "kernel_ms": 0.281859,
            "trials": {"median_ms": 0.2815, "p20_ms": 0.2811, "p80_ms": 0.2822, "trials": 5,
                       "iters": 100},
            "watchdog": "ok", "metric": "HBM GB/s", "value": 5708.1,
            "unit": "TFLOP/s" if ffn else "GB/s", "bytes_per_call": 1610612736,
            "roofline": roof, "clock_MHz": 1553.0 if ffn else None,
            "variants_GBps": {f"split{p}": 5000.0 + p for p in (2, 4, 8, 16, 32)},
            "cpu_baseline": {"value": 6.185, "unit": "GB/s", "cores": 16, "affinity_cores": 16,
                             "cgroup_cpu_quota": 16, "kind": "port",
                             "sample": "2048 of 2048 rows x 65536 cols, median of 50 runs"}}


def test_the_line_with_every_suite_entry_fits_the_kept_tail():
    names = list(hip_lib.HIP_LAUNCHERS)
    assert set(C1_C5) <= set(names)
    suite = {n: bench.compact(synthetic_entry(n, n.startswith("ffn"))) for n in names
             if n != "layernorm_fwd"}
    head = synthetic_entry("layernorm_fwd", False)
    line = {"metric": "m" * 70, "value": head["value"], "unit": "GB/s", "n_gpus": 1,
            "steps": 100, "warmup": 10, "settle_ms": 100.0, "ms_per_step": 0.047,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "d" * 56, "config": {"workload": "layernorm_fwd", "rows": 2048,
                                         "cols": 32768, "device": "x" * 24, "arch": "y" * 22,
                                         "cus": 256, "buffer_sets": 3},
            "kernel_ms": head["kernel_ms"], "trials": head["trials"], "watchdog": "ok",
            "roofline": head["roofline"], "cpu_baseline": head["cpu_baseline"], "suite": suite,
            "detail": "gpurun_out/bench_detail.json"}
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) < 7000, len(text)
    back = json.loads(text)
    for name in C1_C5:
        if name == "layernorm_fwd":
            continue
        entry = back["suite"][name]
        assert {"ms", "value", "unit", "frac", "frac_median", "ceiling_frac"} <= set(entry)
        assert "variants_GBps" not in entry and "trials" not in entry
    assert back["suite"]["ffn"]["clock_MHz"] == 1553.0
    assert back["suite"]["rmsnorm_bwd"]["traffic_ratio"] == round(1613000000 / 1610612736, 3)


def test_traffic_is_reported_only_while_the_sources_are_unchanged(tmp_path, monkeypatch):
    now = source_fingerprints()
    kernels = {k: {"fetch_bytes": 2 * 10**8, "write_bytes": 10**8, "dispatches": 4}
               for k in bench.CALL_KERNELS["rmsnorm_bwd"][1]}
    current = tmp_path / "current.json"
    current.write_text(json.dumps({"commit": "cafe", "sources": now, "kernels": kernels}))
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", current)
    nbytes, note = bench.measured_traffic("rmsnorm_bwd")
    assert nbytes == 6 * 10**8 and note == "PMC at cafe"

    stale = dict(now)
    stale["rmsnorm.hip"] = "0" * 16
    old = tmp_path / "stale.json"
    old.write_text(json.dumps({"commit": "beef", "sources": stale, "kernels": kernels}))
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", old)
    nbytes, note = bench.measured_traffic("rmsnorm_bwd")
    assert nbytes is None and note.startswith("stale: rmsnorm.hip changed")

    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", tmp_path / "missing.json")
    assert bench.measured_traffic("rmsnorm_bwd") == (None, "no PMC summary")


@pytest.mark.parametrize("name", ["rmsnorm_fwd", "rmsnorm_bwd", "layernorm_backward_bf16"])
def test_call_kernels_name_the_group_pipelines_auto_launches(name):
    """The kernel names the PMC summary is looked up by are the template
    instances the library's AUTO path launches at the BASELINE shape (in a
    shape table, or instantiated where the launch takes it)."""
    source, kernels = bench.CALL_KERNELS[name]
    text = (ROOT / "credit_amd" / "csrc" / source).read_text()
    group = [k for k in kernels if "group_kernel" in k]
    assert group, kernels
    for k in group:
        assert "{" + k + "," in text or "fn = " + k + ";" in text, f"{k} is not in {source}"
