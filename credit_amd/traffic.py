"""Per-kernel HBM traffic from rocprofv3 counter runs.

``rocprofv3 --pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` (one counter per run)
write ``*_counter_collection.csv`` with one row per dispatch; the values are
KiB.  On gfx950 the raw FETCH_SIZE reads half of the bytes a kernel fetches
and WRITE_SIZE reads all of them, so each counter is scaled by what it reads
for a stream kernel of known size (``python -m credit_amd.profile --only
hbm_copy --hbm-bytes B``: every ``mb_stream_kernel<1, 1, ...>`` dispatch
reads B bytes and writes B bytes).

    python -m credit_amd.traffic --fetch F.csv --write W.csv \\
        --copy-fetch CF.csv --copy-write CW.csv --copy-bytes B --json out.json

The JSON maps a short kernel name (template arguments kept, namespaces and
parameter lists dropped) to its mean fetched and written bytes per dispatch,
and records what it was measured on: the commit and a SHA-256 prefix of
every kernel source under credit_amd/csrc.  bench.py reports a workload's
sum as ``roofline.traffic`` only while the sources its kernels are built
from still hash the same; after a kernel change the figure is stale and is
reported as null until the counters are collected again.
"""
from __future__ import annotations

import argparse
import collections
import csv
import hashlib
import json
import subprocess
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"
# Headers every kernel source includes: a change there can change any kernel.
SHARED_SOURCES = ("common.hpp", "api_internal.hpp", "slices.hpp")


def source_fingerprints(csrc: Path = CSRC) -> dict[str, str]:
    """SHA-256 prefix (16 hex digits) of every .hip/.hpp file under csrc."""
    out = {}
    for path in sorted(csrc.iterdir()):
        if path.suffix in (".hip", ".hpp"):
            out[path.name] = hashlib.sha256(path.read_bytes()).hexdigest()[:16]
    return out


def sources_unchanged(stamped: dict[str, str], source: str, csrc: Path = CSRC) -> bool:
    """True when `source` and the shared headers hash as they did when the
    counters were collected (`stamped` = the summary's "sources")."""
    now = source_fingerprints(csrc)
    return all(name in stamped and stamped[name] == now.get(name)
               for name in (source, *SHARED_SOURCES))


def current_commit() -> str | None:
    try:
        out = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], capture_output=True,
                             text=True, cwd=CSRC, check=True)
        return out.stdout.strip() or None
    except (OSError, subprocess.CalledProcessError):
        return None


def short_name(kernel: str) -> str:
    """'void credit::(anonymous namespace)::f<512, 8>(args)' -> 'f<512, 8>'."""
    name = kernel.strip().replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):  # drop the parameter list (first '(' outside <>)
        depth += (ch == "<") - (ch == ">")
        if ch == "(" and depth == 0:
            name = name[:i]
            break
    head, sep, tail = name.partition("<")
    return head.split("::")[-1] + sep + tail


def per_kernel_kib(path: str | Path) -> dict[str, tuple[float, int]]:
    """Mean counter value (KiB) per dispatch and dispatch count, by kernel."""
    acc: dict[str, list[float]] = collections.defaultdict(list)
    with open(path, newline="") as fh:
        for row in csv.DictReader(fh):
            acc[short_name(row["Kernel_Name"])].append(float(row["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in acc.items()}


def copy_scale(path: str | Path, copy_bytes: int) -> float:
    """Bytes per counted KiB, from the 1:1 stream dispatches of a known size."""
    vals = [kib for name, (kib, _) in per_kernel_kib(path).items()
            if name.startswith("mb_stream_kernel<1, 1,")]
    if not vals:
        raise RuntimeError(f"{path}: no mb_stream_kernel<1, 1, ...> dispatches")
    return copy_bytes / (sum(vals) / len(vals))


def summarize(fetch: str, write: str, copy_fetch: str, copy_write: str,
              copy_bytes: int, commit: str | None = None) -> dict:
    fs = copy_scale(copy_fetch, copy_bytes)
    ws = copy_scale(copy_write, copy_bytes)
    f = per_kernel_kib(fetch)
    w = per_kernel_kib(write)
    kernels = {}
    for name in sorted(set(f) | set(w)):
        fk = f.get(name, (0.0, 0))
        wk = w.get(name, (0.0, 0))
        kernels[name] = {"fetch_bytes": round(fk[0] * fs), "write_bytes": round(wk[0] * ws),
                         "dispatches": max(fk[1], wk[1])}
    return {"fetch_bytes_per_kib": fs, "write_bytes_per_kib": ws, "copy_bytes": copy_bytes,
            "commit": commit if commit is not None else current_commit(),
            "sources": source_fingerprints(), "kernels": kernels}


def kernel_stats(path: str | Path) -> dict[str, dict[str, float]]:
    """rocprofv3 ``--stats`` kernel summary (``*_kernel_stats.csv``) by short
    kernel name: calls and average / min / max duration in microseconds."""
    out: dict[str, dict[str, float]] = {}
    with open(path, newline="") as fh:
        for row in csv.DictReader(fh):
            out[short_name(row["Name"])] = {
                "calls": int(row["Calls"]),
                "avg_us": float(row["AverageNs"]) / 1e3,
                "min_us": float(row["MinNs"]) / 1e3,
                "max_us": float(row["MaxNs"]) / 1e3,
            }
    return out


def markdown_table(stats: dict[str, dict[str, float]], traffic: dict) -> str:
    """One row per kernel of the trace: calls, durations and, where the PMC
    runs saw the kernel, its HBM fetch and write in MB per dispatch."""
    lines = ["| kernel | calls | avg us | min us | max us | HBM fetch MB | HBM write MB |",
             "|---|---|---|---|---|---|---|"]
    kern = traffic.get("kernels", {})
    for name in sorted(stats, key=lambda n: -stats[n]["avg_us"] * stats[n]["calls"]):
        st = stats[name]
        tr = kern.get(name)
        fetch = f"{tr['fetch_bytes'] / 1e6:.1f}" if tr else "-"
        write = f"{tr['write_bytes'] / 1e6:.1f}" if tr else "-"
        lines.append(f"| `{name}` | {st['calls']} | {st['avg_us']:.1f} | {st['min_us']:.1f} | "
                     f"{st['max_us']:.1f} | {fetch} | {write} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--copy-fetch", required=True)
    ap.add_argument("--copy-write", required=True)
    ap.add_argument("--copy-bytes", type=int, required=True)
    ap.add_argument("--json", required=True)
    ap.add_argument("--commit", help="commit the counters were collected at (default: git HEAD)")
    ap.add_argument("--stats", help="rocprofv3 --stats kernel summary CSV of the same workload")
    ap.add_argument("--markdown", help="write the per-kernel trace + traffic table here")
    args = ap.parse_args(argv)
    out = summarize(args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_bytes,
                    args.commit)
    Path(args.json).write_text(json.dumps(out, indent=1) + "\n")
    if args.markdown:
        if not args.stats:
            ap.error("--markdown needs --stats")
        Path(args.markdown).write_text(markdown_table(kernel_stats(args.stats), out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
