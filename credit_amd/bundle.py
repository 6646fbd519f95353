"""Result bundles of the split sweep: typed tables on disk.

A bundle is the directory ``credit_amd.runner.run_suite`` writes:

* ``metadata.json``   -- device, configuration, calibrated profile, aggregate;
* ``raw.csv``         -- one row per (workload, rows, cols, variant, split);
* ``control.csv``     -- measured split-barrier overhead per (rows, P, barriers);
* ``summary.csv``     -- one row per (workload, rows, cols) point: best
                         no-split variant, best split, the model's verdict;
* ``cluster_sweep.csv`` -- one row per split factor of every point, with the
                         cost model's terms, its predicted traffic and (once
                         credit_amd.counters merged a counter pass) the
                         measured HBM bytes and L2 requests beside them;
* ``REPORT.md``       -- credit_amd.report.

The column sets of summary.csv and cluster_sweep.csv are the contract the
reference's bundles carry (dsmem_eval/runner.py:504-618) with this build's
gfx950 model terms.  Every table has a fixed schema here -- column names and
types, in file order -- so a bundle written by one version reads back with
the same types in another, and a column added to a row without a schema
entry is an error rather than a silently different file.  Values are encoded
as text: ints and floats by ``repr`` (NaN as ``nan``), booleans as
``True``/``False``, a missing value as the empty string (read back as None).
"""
from __future__ import annotations

import csv
import dataclasses
import json
import math
import os
import tempfile
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Iterable

from .cost_model import ModelEstimate

Schema = tuple[tuple[str, type], ...]

RAW: Schema = (
    ("workload", str), ("rows", int), ("cols", int), ("variant", str), ("split", int),
    ("correct", bool), ("ms", float), ("p20_ms", float), ("p80_ms", float), ("samples", int),
    ("error", str), ("threads", int), ("lds_bytes", int), ("per_cu", int), ("dispensers", int),
)

CONTROL: Schema = (("workload", str), ("cols", int), ("rows", int), ("split", int),
                   ("barriers", int), ("threads", int), ("lds_bytes", int), ("per_cu", int),
                   ("overhead_ms", float))

SUMMARY: Schema = (
    ("workload", str), ("label", str), ("category", str), ("rows", int), ("cols", int),
    ("block_variant", str), ("block_ms", float), ("block_p20_ms", float),
    ("block_p80_ms", float), ("split_ms", float), ("measured_split", int),
    ("split_vs_block", float), ("block_gbps", float), ("split_gbps", float),
    ("predicted_split", int), ("model_version", str), ("predicted_delta_ms", float),
    ("predicted_profitable", bool), ("measured_profitable", bool), ("model_correct", bool),
    ("all_variants_correct", bool),
)

_ESTIMATE_TYPES = {float: float, bool: bool, "float": float, "bool": bool}
SWEEP: Schema = (
    ("workload", str), ("rows", int), ("cols", int), ("split", int),
    ("staged_bytes_per_workgroup", int), ("split_ms", float), ("split_p20_ms", float),
    ("split_p80_ms", float), ("control_overhead_ms", float), ("model_version", str),
    *((f.name, _ESTIMATE_TYPES[f.type]) for f in dataclasses.fields(ModelEstimate)),
    ("measured_delta_vs_block_ms", float), ("measured_profitable_vs_block", bool),
    # cost_model.predict_traffic, and beside it the counters of one call of
    # the same variant (credit_amd.counters; empty until merged).
    ("predicted_hbm_bytes", float), ("predicted_block_hbm_bytes", float),
    ("predicted_l2_requests", float), ("predicted_lds_bytes", float),
    ("measured_hbm_bytes", float), ("measured_block_hbm_bytes", float),
    ("measured_l2_requests", float), ("measured_lds_instructions", float),
    ("counter_source", str),
)

TABLES: dict[str, Schema] = {
    "raw.csv": RAW,
    "control.csv": CONTROL,
    "summary.csv": SUMMARY,
    "cluster_sweep.csv": SWEEP,
}


def encode(value: Any, kind: type) -> str:
    if value is None:
        return ""
    if kind is bool:
        return "True" if bool(value) else "False"
    if kind is float:
        v = float(value)
        return "nan" if math.isnan(v) else repr(v)
    if kind is int:
        return str(int(value))
    return str(value)


def decode(text: str | None, kind: type) -> Any:
    if text is None or text == "":
        return None
    if kind is bool:
        low = text.strip().lower()
        if low in ("true", "1"):
            return True
        if low in ("false", "0"):
            return False
        raise ValueError(f"not a boolean: {text!r}")
    if kind is int:
        return int(float(text))
    if kind is float:
        return float(text)
    return text


def _atomic_write(path: Path, text: str) -> None:
    """Write beside the target, then rename over it: a reader never sees a
    half-written file."""
    path.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(dir=path.parent, prefix=f".{path.name}.")
    try:
        with os.fdopen(fd, "w", encoding="utf-8", newline="") as fh:
            fh.write(text)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise


def write_table(path: Path, rows: Iterable[dict[str, Any]], schema: Schema) -> None:
    names = [n for n, _ in schema]
    kinds = dict(schema)
    lines: list[list[str]] = [names]
    for row in rows:
        extra = sorted(set(row) - set(kinds))
        if extra:
            raise ValueError(f"{path.name}: columns {extra} are not in its schema")
        lines.append([encode(row.get(n), kinds[n]) for n in names])
    from io import StringIO

    buf = StringIO()
    csv.writer(buf, lineterminator="\n").writerows(lines)
    _atomic_write(Path(path), buf.getvalue())


def read_table(path: Path, schema: Schema) -> list[dict[str, Any]]:
    """Typed rows.  Columns the schema lacks (a newer writer) are kept as
    text; schema columns the file lacks (an older writer) read as None."""
    kinds = dict(schema)
    with Path(path).open(newline="", encoding="utf-8") as fh:
        reader = csv.DictReader(fh)
        out = []
        for raw in reader:
            row = {n: decode(raw.get(n), k) for n, k in schema}
            row.update({n: v for n, v in raw.items() if n not in kinds})
            out.append(row)
    return out


@dataclass
class Bundle:
    root: Path
    metadata: dict[str, Any]
    summary: list[dict[str, Any]] = field(default_factory=list)
    sweep: list[dict[str, Any]] = field(default_factory=list)

    @classmethod
    def load(cls, root: Path) -> "Bundle":
        root = Path(root).resolve()
        needed = ("metadata.json", "summary.csv", "cluster_sweep.csv")
        missing = [n for n in needed if not (root / n).is_file()]
        if missing:
            raise FileNotFoundError(f"{root}: missing {', '.join(missing)}")
        return cls(root=root,
                   metadata=json.loads((root / "metadata.json").read_text(encoding="utf-8")),
                   summary=read_table(root / "summary.csv", SUMMARY),
                   sweep=read_table(root / "cluster_sweep.csv", SWEEP))

    def save_tables(self) -> None:
        write_table(self.root / "summary.csv", self.summary, SUMMARY)
        write_table(self.root / "cluster_sweep.csv", self.sweep, SWEEP)

    def save_metadata(self) -> None:
        _atomic_write(self.root / "metadata.json", json.dumps(self.metadata, indent=2) + "\n")
