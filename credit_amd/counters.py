"""Hardware counters of the split sweep, beside the cost model's predicted traffic.

The sweep (credit_amd.runner) times every variant over many calls; counters
are collected in a run of their own, one call per (point, variant), under
rocprofv3 -- one counter per run, as the hardware allows:

    python -m credit_amd.counters pass --plan P.json [sweep options]      # under rocprofv3 --pmc C
    python -m credit_amd.counters merge BUNDLE --plan P.json \\
        --fetch F.csv --write W.csv --copy-fetch CF.csv --copy-write CW.csv \\
        --copy-bytes B [--l2-requests T.csv] [--lds-instructions L.csv]

``pass`` issues, for every plan entry, a marker dispatch -- a bf16 transpose
of a 64 x 64 (i + 2) tile, whose grid of i + 2 workgroups names entry i --
followed by one call of the entry's variant; every dispatch up to the next
marker belongs to that entry (a call may launch more than one kernel).  A
one-workgroup marker precedes the input preparation of every point, so the
dispatches that preparation makes belong to no entry.
``merge`` sums each counter over an entry's dispatches, scales FETCH_SIZE and
WRITE_SIZE by what they read for a copy kernel of known size
(credit_amd.traffic.copy_scale), and writes the results into the bundle's
cluster_sweep.csv beside cost_model.predict_traffic's columns:
measured_hbm_bytes (split variant), measured_block_hbm_bytes (the point's
best no-split variant), measured_l2_requests (TCC_REQ_sum, split) and
measured_lds_instructions (SQ_INSTS_LDS, split: wave-level LDS instructions
of the call, beside predicted_lds_bytes, which prices only the exchange
copies; the kernels' block reductions and LDS rings are the rest).  It
also writes counters.csv, one row per plan entry, and TRAFFIC.md, the
measured / predicted ratios per workload.  The plan is a pure
function of the sweep options, so it names the same rows as the timed sweep.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import math
from pathlib import Path
from typing import Any

from .traffic import copy_scale, short_name

MARKER = "transpose_bf16_kernel"
MARKER_LANES = 256  # threads per marker workgroup


def build_plan(workloads, n_values, splits, tensor_bytes) -> list[dict[str, Any]]:
    """Entries (workload, rows, cols, variant, split) in issue order: every
    variant the timed sweep runs at every point."""
    from .runner import sweep_rows, variant_list
    from .workloads import WORKLOADS

    plan = []
    for name in workloads:
        spec = WORKLOADS[name]
        for cols in n_values:
            rows = sweep_rows(spec, cols, tensor_bytes)
            for variant, split in variant_list(spec, cols, tuple(splits)):
                plan.append({"index": len(plan), "workload": name, "rows": rows, "cols": cols,
                             "variant": variant, "split": split})
    return plan


def run_pass(plan: list[dict[str, Any]]) -> list[dict[str, Any]]:
    """One marker and one call per entry (GPU).  Returns the entries with
    the call's status ("ok" or the library error)."""
    import torch

    from . import hip_lib
    from .workloads import WORKLOADS

    dev = torch.device("cuda:0")
    hip_lib.load_library()
    # Marker operands, allocated (and zero-filled) before the first marker.
    longest = 64 * (len(plan) + 2)
    msrc = torch.zeros(64 * longest, dtype=torch.bfloat16, device=dev)
    mdst = torch.empty(64 * longest, dtype=torch.bfloat16, device=dev)

    def marker(blocks: int) -> None:
        n = 64 * blocks
        hip_lib.transpose(msrc[: 64 * n].view(64, n), mdst[: 64 * n].view(n, 64))

    out = []
    point = None
    sets = outs = None
    for e in plan:
        key = (e["workload"], e["rows"], e["cols"])
        if key != point:
            marker(1)  # what follows until the next entry's marker is no entry's
            sets = outs = None
            torch.cuda.empty_cache()
            spec = WORKLOADS[e["workload"]]
            sets = hip_lib.prepare_inputs(e["workload"],
                                          spec.make_inputs(e["rows"], e["cols"],
                                                           seed=1234 + e["cols"]), dev)
            outs = hip_lib.allocate_outputs(e["workload"], sets)
            point = key
            print(f"counters {key[0]}: rows={key[1]} cols={key[2]}", flush=True)
        torch.cuda.synchronize()
        marker(e["index"] + 2)
        status = "ok"
        try:
            hip_lib.HIP_LAUNCHERS[e["workload"]](sets, outs,
                                                 hip_lib.LaunchConfig(e["variant"], e["split"]))
            torch.cuda.synchronize()
            hip_lib.check_watchdog()
        except hip_lib.CreditError as err:
            status = f"{err.status}: {err}"
            torch.cuda.synchronize()
        out.append({**e, "status": status})
    return out


def entry_sums(counter_csv: str | Path) -> dict[int, dict[str, float]]:
    """Per plan entry, each counter summed over the dispatches between its
    marker and the next (markers themselves excluded)."""
    by_dispatch: dict[int, dict[str, Any]] = {}
    with open(counter_csv, newline="") as fh:
        for row in csv.DictReader(fh):
            d = by_dispatch.setdefault(int(row["Dispatch_Id"]), {
                "name": short_name(row["Kernel_Name"]), "grid": int(row["Grid_Size"]),
                "counters": collections.defaultdict(float)})
            d["counters"][row["Counter_Name"]] += float(row["Counter_Value"])
    sums: dict[int, dict[str, float]] = {}
    current = None
    for _, d in sorted(by_dispatch.items()):
        if d["name"] == MARKER and d["grid"] % MARKER_LANES == 0:
            blocks = d["grid"] // MARKER_LANES
            current = blocks - 2 if blocks >= 2 else None
            if current is not None:
                sums.setdefault(current, collections.defaultdict(float))
            continue
        if current is None:
            continue
        for name, value in d["counters"].items():
            sums[current][name] += value
    return sums


def merge(bundle_dir: Path, plan_path: Path, fetch: str, write: str, copy_fetch: str,
          copy_write: str, copy_bytes: int, l2_requests: str | None = None,
          lds_instructions: str | None = None) -> dict[str, Any]:
    from . import bundle as bundle_mod

    plan = json.loads(Path(plan_path).read_text())
    entries = plan["entries"]
    fs, ws = copy_scale(copy_fetch, copy_bytes), copy_scale(copy_write, copy_bytes)
    f, w = entry_sums(fetch), entry_sums(write)
    t = entry_sums(l2_requests) if l2_requests else {}
    ld = entry_sums(lds_instructions) if lds_instructions else {}
    rows_out = []
    measured: dict[tuple[str, int, int, str, int], dict[str, float]] = {}
    for e in entries:
        i = e["index"]
        hbm = (f.get(i, {}).get("FETCH_SIZE", math.nan) * fs +
               w.get(i, {}).get("WRITE_SIZE", math.nan) * ws)
        req = t.get(i, {}).get("TCC_REQ_sum", math.nan) if t else math.nan
        lds = ld.get(i, {}).get("SQ_INSTS_LDS", math.nan) if ld else math.nan
        key = (e["workload"], e["rows"], e["cols"], e["variant"], e["split"])
        measured[key] = {"hbm": hbm, "l2": req, "lds": lds}
        rows_out.append({**{k: e[k] for k in ("index", "workload", "rows", "cols", "variant",
                                              "split")},
                         "status": e.get("status", ""), "hbm_bytes": hbm, "l2_requests": req,
                         "lds_instructions": lds})
    b = bundle_mod.Bundle.load(bundle_dir)
    block_of = {(r["workload"], r["rows"], r["cols"]): r["block_variant"] for r in b.summary}
    source = f"counter pass {Path(plan_path).name}"
    filled = 0
    for r in b.sweep:
        pt = (r["workload"], r["rows"], r["cols"])
        m = measured.get((*pt, "split", r["split"]))
        if m is None:
            continue
        blk = measured.get((*pt, block_of.get(pt, "read"), 0), {"hbm": math.nan})
        r.update(measured_hbm_bytes=m["hbm"], measured_block_hbm_bytes=blk["hbm"],
                 measured_l2_requests=m["l2"], measured_lds_instructions=m["lds"],
                 counter_source=source)
        filled += 1
    b.save_tables()
    with (Path(bundle_dir) / "counters.csv").open("w", newline="") as fh:
        wr = csv.DictWriter(fh, fieldnames=list(rows_out[0]))
        wr.writeheader()
        wr.writerows(rows_out)
    return {"entries": len(entries), "sweep_rows_filled": filled,
            "fetch_bytes_per_kib": fs, "write_bytes_per_kib": ws}


def agreement(bundle_dir: Path) -> list[dict[str, Any]]:
    """Measured / predicted per sweep row that carries counters."""
    from . import bundle as bundle_mod

    out = []
    for r in bundle_mod.Bundle.load(bundle_dir).sweep:
        if r.get("measured_hbm_bytes") is None or not math.isfinite(r["measured_hbm_bytes"]):
            continue
        out.append({
            "workload": r["workload"], "rows": r["rows"], "cols": r["cols"], "split": r["split"],
            "hbm_ratio": r["measured_hbm_bytes"] / r["predicted_hbm_bytes"],
            "block_hbm_ratio": (r["measured_block_hbm_bytes"] / r["predicted_block_hbm_bytes"]
                                if r.get("measured_block_hbm_bytes") else math.nan),
            "l2_ratio": (r["measured_l2_requests"] / r["predicted_l2_requests"]
                         if r.get("measured_l2_requests") else math.nan),
            # per row and member: the LDS instructions counted, the exchange
            # bytes the model prices into LDS
            "lds_insts_per_row_member": (r["measured_lds_instructions"] / (r["rows"] * r["split"])
                                         if r.get("measured_lds_instructions") else math.nan),
            "lds_bytes_per_row_member": (r["predicted_lds_bytes"] / (r["rows"] * r["split"])
                                         if r.get("predicted_lds_bytes") is not None else math.nan),
        })
    return out


def traffic_report(bundle_dir: Path) -> str:
    """TRAFFIC.md: per workload, measured / predicted HBM bytes of the
    split and no-split variants and L2 requests of the split, over the
    sweep rows that carry counters."""
    import statistics

    rows = agreement(bundle_dir)
    by: dict[str, list[dict[str, Any]]] = collections.defaultdict(list)
    for r in rows:
        by[r["workload"]].append(r)

    def span(vals, fmt=".3f"):
        v = [x for x in vals if math.isfinite(x)]
        if not v:
            return "-"
        return f"{statistics.median(v):{fmt}} [{min(v):{fmt}}, {max(v):{fmt}}]"

    lines = ["# Counters against the cost model's traffic", "",
             "measured / predicted per sweep row (median [min, max]); HBM = scaled FETCH_SIZE +"
             " WRITE_SIZE of one call, L2 = TCC_REQ_sum. LDS: SQ_INSTS_LDS (wave instructions) per"
             " row and member, beside the exchange bytes per row and member the model copies into"
             " LDS (not a ratio: the counted instructions include the block reductions and LDS"
             " rings the model does not price).", "",
             "| workload | rows | split HBM | no-split HBM | split L2 requests |"
             " split LDS instr. / row / member | predicted LDS B / row / member |",
             "|---|---:|---|---|---|---|---|"]
    for name in sorted(by):
        rs = by[name]
        lines.append(f"| {name} | {len(rs)} | {span([r['hbm_ratio'] for r in rs])} | "
                     f"{span([r['block_hbm_ratio'] for r in rs])} | "
                     f"{span([r['l2_ratio'] for r in rs])} | "
                     f"{span([r['lds_insts_per_row_member'] for r in rs], '.0f')} | "
                     f"{span([r['lds_bytes_per_row_member'] for r in rs], '.0f')} |")
    within = sum(1 for r in rows if abs(r["hbm_ratio"] - 1.0) < 0.05)
    within_b = sum(1 for r in rows
                   if math.isfinite(r["block_hbm_ratio"]) and abs(r["block_hbm_ratio"] - 1.0) < 0.05)
    lines += ["", f"Split HBM bytes within 5% of the prediction: {within}/{len(rows)} rows; "
                  f"no-split: {within_b}/{len(rows)}."]
    text = "\n".join(lines) + "\n"
    (Path(bundle_dir) / "TRAFFIC.md").write_text(text)
    return text


def main(argv=None) -> int:
    from .runner import DEFAULT_N_VALUES, DEFAULT_SPLITS, DEFAULT_TENSOR_BYTES, SWEEP_WORKLOADS

    def ints(v: str) -> tuple[int, ...]:
        return tuple(int(x) for x in v.split(",") if x.strip())

    ap = argparse.ArgumentParser(description="split-sweep hardware counters")
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("pass", help="one marker + one call per (point, variant); run under rocprofv3")
    p.add_argument("--plan", type=Path, required=True, help="where to write the plan (JSON)")
    p.add_argument("--workloads", default="all")
    p.add_argument("--n-values", type=ints, default=DEFAULT_N_VALUES)
    p.add_argument("--splits", type=ints, default=DEFAULT_SPLITS)
    p.add_argument("--tensor-bytes", type=int, default=DEFAULT_TENSOR_BYTES)
    m = sub.add_parser("merge", help="sum a pass's counters per entry into a sweep bundle")
    m.add_argument("bundle", type=Path)
    m.add_argument("--plan", type=Path, required=True)
    m.add_argument("--fetch", required=True)
    m.add_argument("--write", required=True)
    m.add_argument("--copy-fetch", required=True)
    m.add_argument("--copy-write", required=True)
    m.add_argument("--copy-bytes", type=int, required=True)
    m.add_argument("--l2-requests")
    m.add_argument("--lds-instructions", help="SQ_INSTS_LDS counter CSV of a pass")
    args = ap.parse_args(argv)
    if args.cmd == "pass":
        workloads = SWEEP_WORKLOADS if args.workloads == "all" else tuple(
            x.strip() for x in args.workloads.split(",") if x.strip())
        plan = build_plan(workloads, args.n_values, args.splits, args.tensor_bytes)
        done = run_pass(plan)
        args.plan.write_text(json.dumps({"tensor_bytes": args.tensor_bytes, "entries": done},
                                        indent=1) + "\n")
        print(f"counter pass: {len(done)} entries -> {args.plan}", flush=True)
        return 0
    res = merge(args.bundle, args.plan, args.fetch, args.write, args.copy_fetch, args.copy_write,
                args.copy_bytes, args.l2_requests, args.lds_instructions)
    print(json.dumps(res))
    print(traffic_report(args.bundle))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
