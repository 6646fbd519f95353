"""gfx950 calibration: run the microbenchmarks and build a DeviceProfile.

The reference runs ``build/primitive_benchmark`` in a subprocess and parses
its human-readable stdout with regular expressions
(dsmem_eval/profile.py:27-103, dsmem_eval/runner.py:248-255), then folds the
numbers into a ``DeviceProfile`` (dsmem_eval/profile.py:106-126).  Here the
microbenchmarks are calls into ``libcredit_hip.so`` (``credit_microbench``,
``credit_control_overhead``) and the profile is built from their results
directly.  ``format_profile_text`` / ``parse_profile_text`` keep a text form
with one ``Key: value unit`` line per measurement, so a saved calibration can
be re-read without a GPU, as the reference re-reads ``primitive_stdout.txt``.

CDNA4 has no distributed shared memory.  The reference's DSMEM figures
(cluster sync latency, DSMEM store throughput, store-visibility round trip;
src/primitive_benchmark.cu:236-566) are replaced by the costs of the
split-row exchange this library uses: device-scope atomic round trips
between two workgroups on one XCD and on two XCDs, and the time of a
P-member arrival barrier inside a cooperative grid.
"""
from __future__ import annotations

import argparse
import json
import re
import sys
from dataclasses import asdict
from typing import Any

from . import hip_lib
from .cost_model import DeviceProfile

FLOAT = r"([0-9]+(?:\.[0-9]+)?(?:[eE][-+]?[0-9]+)?)"

# (key in the parsed dict, text label, unit) -- the text protocol.
TEXT_KEYS: tuple[tuple[str, str, str], ...] = (
    ("clock_ghz", "Clock frequency", "GHz"),
    ("cu_count", "CU count", ""),
    ("xcd_count", "XCD count", ""),
    ("lds_bytes_per_cu", "LDS per CU", "bytes"),
    ("max_lds_bytes_per_block", "LDS per workgroup", "bytes"),
    ("l2_capacity_bytes", "L2 capacity", "bytes"),
    ("l1_latency_cycles", "L1 read latency", "cycles"),
    ("l2_latency_cycles", "L2 read latency", "cycles"),
    ("mall_latency_cycles", "MALL read latency", "cycles"),
    ("hbm_latency_cycles", "HBM read latency", "cycles"),
    ("hbm_read_gbps", "HBM read bandwidth", "GB/s"),
    ("hbm_write_gbps", "HBM write bandwidth", "GB/s"),
    ("hbm_copy_gbps", "HBM copy bandwidth", "GB/s"),
    ("l1_read_bytes_per_cycle_cu", "L1 read bandwidth", "B/cycle/CU"),
    ("l2_read_bytes_per_cycle_xcd", "L2 read bandwidth", "B/cycle/XCD"),
    ("l2_read_gbps", "L2 read bandwidth (device)", "GB/s"),
    ("lds_read_bytes_per_cycle_cu", "LDS read throughput", "B/cycle/CU"),
    ("lds_write_bytes_per_cycle_cu", "LDS write throughput", "B/cycle/CU"),
    ("exchange_roundtrip_cycles_xcd", "Exchange round trip same XCD", "cycles"),
    ("exchange_roundtrip_cycles_cross", "Exchange round trip cross XCD", "cycles"),
    ("slot_store_bytes_per_cycle_wg", "Exchange slot store throughput", "B/cycle/WG"),
    ("slot_store_gbps", "Exchange slot store throughput (device)", "GB/s"),
    ("ticket_cycles_private", "Ticket draw private line", "cycles"),
    ("ticket_cycles_shared", "Ticket draw shared line", "cycles"),
    ("mfma_bf16_tflops", "MFMA bf16 rate", "TFLOP/s"),
    ("mfma_clock_mhz", "MFMA shader clock", "MHz"),
)


def run_microbenchmarks(hbm_bytes: int = 1 << 30, iters: int = 20) -> dict[str, Any]:
    """Run every gfx950 microbenchmark once on device 0 (the current device)."""
    info = hip_lib.query_device(0)
    clock_mhz = hip_lib.microbench("clock")[0]
    lat = hip_lib.microbench("latency", 0, 20000, 4)
    read = hip_lib.microbench("hbm_read", hbm_bytes, iters)
    write = hip_lib.microbench("hbm_write", hbm_bytes, iters)
    copy = hip_lib.microbench("hbm_copy", hbm_bytes, iters)
    lds_r = hip_lib.microbench("lds_read", 0, 4096)[0]
    lds_w = hip_lib.microbench("lds_write", 0, 4096)[0]
    rt = hip_lib.microbench("exchange_roundtrip", 0, 2000, 2)
    cache = hip_lib.microbench("cache_read", 0, 64, 3)
    xput = hip_lib.microbench("exchange_throughput", 0, 4096, 4)
    mfma = hip_lib.microbench("mfma_bf16", 0, 20000, 6)
    return {
        "name": info["name"],
        "arch": info["arch"],
        "clock_ghz": clock_mhz / 1000.0,
        "cu_count": info["cu_count"],
        "xcd_count": info["xcd_count"],
        "lds_bytes_per_cu": info["lds_bytes_per_cu"],
        "max_lds_bytes_per_block": info["lds_bytes_per_block"],
        "l2_capacity_bytes": info["l2_bytes"],
        "l1_latency_cycles": lat[0],
        "l2_latency_cycles": lat[1],
        "mall_latency_cycles": lat[2],
        "hbm_latency_cycles": lat[3],
        "hbm_read_gbps": read[0],
        "hbm_write_gbps": write[0],
        "hbm_copy_gbps": copy[0],
        "hbm_read_shapes_gbps": [v for v in read[1:] if v > 0],
        "hbm_copy_shapes_gbps": [v for v in copy[1:] if v > 0],
        "lds_read_bytes_per_cycle_cu": lds_r,
        "lds_write_bytes_per_cycle_cu": lds_w,
        "exchange_roundtrip_cycles_xcd": rt[0],
        "exchange_roundtrip_cycles_cross": rt[1],
        "l1_read_bytes_per_cycle_cu": cache[0],
        "l2_read_bytes_per_cycle_xcd": cache[1],
        "l2_read_gbps": cache[2],
        "slot_store_bytes_per_cycle_wg": xput[0],
        "slot_store_gbps": xput[1],
        "ticket_cycles_private": xput[2],
        "ticket_cycles_shared": xput[3],
        "mfma_bf16_tflops": mfma[0],
        "mfma_clock_mhz": mfma[1],
    }


# Read:write stream mixes credit_stream_ceiling builds (workloads.py's
# stream_mix of every workload is one of them).
CEILING_MIXES = ((1, 0), (0, 1), (1, 1), (2, 1), (3, 1), (4, 1), (3, 2), (2, 2), (1, 2))


def ceiling_table(sizes: list[int], trials: int = 5, iters: int = 20) -> str:
    """Markdown: best settled GB/s (and its launch shape) per mix and call size."""
    lines = ["| mix (read:write) | " + " | ".join(f"{s / 2**20:.0f} MiB per call" for s in sizes)
             + " |", "|---|" + "---|" * len(sizes)]
    for r, w in CEILING_MIXES:
        cells = []
        for s in sizes:
            c = hip_lib.stream_ceiling(r, w, s, trials=trials, iters=iters, settle_ms=20.0)
            sh = c["shape"]
            cells.append(f"{c['GBps']:.0f} GB/s ({sh['lanes']}x{sh['vectors_per_lane']}, "
                         f"{sh['workgroups_per_cu']}/CU{', nt' if sh['nontemporal_stores'] else ''})")
        lines.append(f"| {r}:{w} | " + " | ".join(cells) + " |")
        print(f"ceiling {r}:{w} done", file=sys.stderr, flush=True)
    # The runtime's own copy (hipMemcpyAsync device to device) at the same
    # 1:1 call sizes, settled and rotated the same way: an independent check
    # of the 1:1 row.
    cells = []
    for s in sizes:
        gbps, ms = hip_lib.microbench("runtime_copy", s // 2, iters, 2)
        cells.append(f"{gbps:.0f} GB/s ({ms * 1e3:.1f} us per call)")
    lines.append("| 1:1, runtime D2D copy | " + " | ".join(cells) + " |")
    return "\n".join(lines) + "\n"


def run_control_sweep(rows: int = 1024, splits=(2, 4, 8, 16), barriers=(1, 2, 3),
                      warmup: int = 3, iters: int = 20) -> list[dict[str, Any]]:
    """credit_control_overhead over (P, barriers) with the plain ticketed
    launch the split kernels use, plus the cooperative launch at one barrier
    for comparison.  Replaces the per-shape build/cluster_control runs of
    dsmem_eval/runner.py:313-347."""
    out = []
    for p in splits:
        for b in barriers:
            for coop in (False, True):
                if coop and b != 1:
                    continue
                plain, split = hip_lib.control_overhead(rows, p, b, warmup, iters, coop)
                out.append({"rows": rows, "split": p, "barriers": b, "cooperative": coop,
                            "plain_ms": plain, "split_ms": split,
                            "overhead_ms": max(split - plain, 0.0)})
    return out


def format_profile_text(parsed: dict[str, Any]) -> str:
    lines = [f"GPU Model: {parsed['name']}"]
    for key, label, unit in TEXT_KEYS:
        value = parsed[key]
        text = f"{value:.6g}" if isinstance(value, float) else str(value)
        lines.append(f"{label}: {text} {unit}".rstrip())
    return "\n".join(lines) + "\n"


def parse_profile_text(text: str) -> dict[str, Any]:
    """Inverse of format_profile_text (the role of
    dsmem_eval/profile.py:27-103).  Raises if a key is missing."""
    m = re.search(r"^GPU Model:\s*(.+)$", text, flags=re.MULTILINE)
    if m is None:
        raise RuntimeError("calibration text does not name the GPU model")
    parsed: dict[str, Any] = {"name": m.group(1).strip()}
    for key, label, _unit in TEXT_KEYS:
        m = re.search(rf"^{re.escape(label)}:\s*{FLOAT}", text, flags=re.MULTILINE)
        if m is None:
            raise RuntimeError(f"calibration text does not report {label}")
        v = float(m.group(1))
        parsed[key] = int(v) if key in ("cu_count", "xcd_count", "lds_bytes_per_cu",
                                        "max_lds_bytes_per_block", "l2_capacity_bytes") else v
    return parsed


def make_device_profile(parsed: dict[str, Any]) -> DeviceProfile:
    """Fold the measurements into the cost model's DeviceProfile
    (dsmem_eval/profile.py:106-126 does this for the DSMEM fields)."""
    return DeviceProfile(
        name=str(parsed["name"]),
        cu_count=int(parsed["cu_count"]),
        xcd_count=int(parsed["xcd_count"]),
        clock_ghz=float(parsed["clock_ghz"]),
        hbm_read_gbps=float(parsed["hbm_read_gbps"]),
        hbm_copy_gbps=float(parsed["hbm_copy_gbps"]),
        l2_capacity_bytes=int(parsed["l2_capacity_bytes"]),
        lds_bytes_per_cu=int(parsed["lds_bytes_per_cu"]),
        max_lds_bytes_per_block=int(parsed["max_lds_bytes_per_block"]),
        lds_read_bytes_per_cycle_cu=float(parsed["lds_read_bytes_per_cycle_cu"]),
        lds_write_bytes_per_cycle_cu=float(parsed["lds_write_bytes_per_cycle_cu"]),
        exchange_roundtrip_cycles=float(parsed["exchange_roundtrip_cycles_xcd"]),
        hbm_latency_cycles=float(parsed["hbm_latency_cycles"]),
    )


def profile_as_dict(profile: DeviceProfile) -> dict[str, Any]:
    return asdict(profile)


def run_ffn_reference(rows: int = 4096, d: int = 8192, f: int = 28672, reps: int = 2,
                      gemm2: bool = False) -> None:
    """The FFN forward (this library's two GEMMs) and the vendor library's GEMM
    of GEMM1's shape (torch.matmul -> hipBLASLt), `reps` times each, on random
    bf16 operands in the nn.Linear layouts; with `gemm2` also the vendor GEMM of
    GEMM2's shape (h @ W2^T).  A workload for per-kernel counter collection
    (rocprofv3 --pmc), not a benchmark."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(rows, d, device=dev, generator=g).bfloat16()
    w1 = (torch.randn(f, d, device=dev, generator=g) / d ** 0.5).bfloat16()
    w2 = (torch.randn(d, f, device=dev, generator=g) / f ** 0.5).bfloat16()
    out = torch.empty_like(x)
    cfg = hip_lib.make_cfg("auto")
    for _ in range(reps):
        hip_lib.ffn(x, w1, w2, out, hip_lib.FFN_EPS, cfg)
    torch.cuda.synchronize()
    for _ in range(reps):
        torch.matmul(x, w1.t())
    torch.cuda.synchronize()
    if gemm2:
        h = torch.randn(rows, f, device=dev, generator=g).bfloat16()
        for _ in range(reps):
            torch.matmul(h, w2.t())
        torch.cuda.synchronize()
    print("ffn reference workload done", flush=True)


def ffn_vs_library(rows: int = 4096, d: int = 8192, f: int = 28672, rounds: int = 2,
                   calls: int = 20) -> list[dict[str, Any]]:
    """Same-process timing of this library's C5 FFN forward against the vendor
    path on the same operands: hipBLASLt (torch.matmul) on GEMM1's and
    GEMM2's shapes, and the unfused torch FFN (rms_norm, matmul, gelu tanh,
    matmul, residual add).  Each line: `calls` calls after 5 warmup calls,
    bracketed by events on torch's current stream, `rounds` times in turn."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(rows, d, device=dev, generator=g).bfloat16()
    w1 = (torch.randn(f, d, device=dev, generator=g) / d ** 0.5).bfloat16()
    w2 = (torch.randn(d, f, device=dev, generator=g) / f ** 0.5).bfloat16()
    h = torch.randn(rows, f, device=dev, generator=g).bfloat16()
    out = torch.empty_like(x)
    cfg = hip_lib.make_cfg("auto")
    gemm = 2.0 * rows * d * f

    def torch_ffn():
        a = torch.nn.functional.rms_norm(x, (d,), eps=hip_lib.FFN_EPS)
        hh = torch.nn.functional.gelu(a @ w1.t(), approximate="tanh")
        return x + hh @ w2.t()

    cases = [("this library's fused FFN", lambda: hip_lib.ffn(x, w1, w2, out, hip_lib.FFN_EPS, cfg),
              2 * gemm),
             ("hipBLASLt, GEMM1 shape (x @ W1^T)", lambda: torch.matmul(x, w1.t()), gemm),
             ("hipBLASLt, GEMM2 shape (h @ W2^T)", lambda: torch.matmul(h, w2.t()), gemm),
             ("torch FFN over hipBLASLt", torch_ffn, 2 * gemm)]
    rows_out = []
    for rnd in range(rounds):
        for name, fn, flop in cases:
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(calls):
                fn()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) / calls * 1e3
            rows_out.append({"round": rnd + 1, "case": name, "us": us,
                             "tflops": flop / us / 1e6})
            print(f"round {rnd + 1}  {name:36s} {us:8.1f} us  {flop / us / 1e6:7.1f} TFLOP/s",
                  flush=True)
    return rows_out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="gfx950 calibration microbenchmarks")
    ap.add_argument("--hbm-bytes", type=int, default=1 << 30)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--control", action="store_true", help="also sweep the barrier overhead")
    ap.add_argument("--json", help="write the measurements (and control sweep) here")
    ap.add_argument("--only", choices=sorted(hip_lib.MICROBENCH),
                    help="run just this microbenchmark (e.g. hbm_copy of --hbm-bytes as the "
                         "known-size reference for PMC byte counters) and print its results")
    ap.add_argument("--ceilings", metavar="BYTES[,BYTES...]",
                    help="settled HBM stream ceilings (credit_stream_ceiling) of every built "
                         "read:write mix at these bytes per call, as a markdown table")
    ap.add_argument("--ffn-reference", action="store_true",
                    help="run the C5 FFN forward twice, then hipBLASLt (torch.matmul) on GEMM1's "
                         "shape twice: the workload of the FFN-against-library counter runs")
    ap.add_argument("--ffn-vs-library", action="store_true",
                    help="time the C5 FFN forward against hipBLASLt's GEMMs of its shapes and "
                         "the unfused torch FFN in one process")
    ap.add_argument("--reps", type=int, default=2, help="calls of each in --ffn-reference")
    ap.add_argument("--gemm2", action="store_true",
                    help="--ffn-reference also runs hipBLASLt on GEMM2's shape")
    args = ap.parse_args(argv)
    import torch  # noqa: F401  (loads the HIP runtime torch uses before the library)

    if args.ffn_vs_library:
        ffn_vs_library()
        return 0
    if args.ffn_reference:
        run_ffn_reference(reps=args.reps, gemm2=args.gemm2)
        return 0
    if args.ceilings:
        sys.stdout.write(ceiling_table([int(b) for b in args.ceilings.split(",") if b.strip()]))
        return 0
    if args.only:
        res = hip_lib.microbench(args.only, args.hbm_bytes, args.iters)
        print(f"{args.only} bytes={args.hbm_bytes} iters={args.iters} results={res}", flush=True)
        return 0

    parsed = run_microbenchmarks(args.hbm_bytes, args.iters)
    sys.stdout.write(format_profile_text(parsed))
    result: dict[str, Any] = {"measurements": parsed,
                              "cost_model_profile": profile_as_dict(make_device_profile(parsed))}
    if args.control:
        result["control"] = run_control_sweep()
        for row in result["control"]:
            print("CONTROL,{rows},{split},{barriers},{cooperative:d},{plain_ms:.6f},{split_ms:.6f},"
                  "{overhead_ms:.6f}".format(**row))
    if args.json:
        with open(args.json, "w", encoding="utf-8") as fh:
            json.dump(result, fh, indent=2)
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
