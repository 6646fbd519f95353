"""Loading the golden fixtures written by make_golden.py."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

DIR = Path(__file__).resolve().parent


def cases() -> list[str]:
    return sorted(p.stem for p in DIR.glob("*.npz"))


def load(case: str):
    """(meta dict, input tensors on the CPU, expected output arrays)."""
    with np.load(DIR / f"{case}.npz", allow_pickle=False) as z:
        meta = json.loads(str(z["meta"]))
        inputs = []
        for i, tag in enumerate(meta["inputs"]):
            a = z[f"in{i}"]
            if tag == "bf16":
                inputs.append(torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16))
            else:
                inputs.append(torch.from_numpy(a.copy()))
        expected = [z[f"out{i}"] for i in range(len(meta["outputs"]))]
    return meta, inputs, expected


def check(got: np.ndarray, want: np.ndarray, spec: dict, what: str) -> None:
    """Compare one output against its fixture under the fixture's check."""
    got = np.asarray(got)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    kind = spec["check"]
    if kind == "exact":
        if want.dtype.kind == "f":
            ok = np.array_equal(got.astype(want.dtype), want, equal_nan=True)
        else:
            ok = np.array_equal(got.astype(want.dtype), want)
        assert ok, f"{what}: not bit-exact ({int((got != want).sum())} elements differ)"
        return
    got = np.asarray(got, dtype=np.float64)
    if kind == "rowmax":
        atol = spec["atol"] * np.abs(want).max(axis=-1, keepdims=True)
        bad = ~(np.abs(got - want) <= atol + spec["rtol"] * np.abs(want))
        assert not bad.any(), (f"{what}: {int(bad.sum())} elements outside rtol {spec['rtol']} / "
                               f"atol {spec['atol']} x row max; worst "
                               f"{np.abs(got - want)[bad].max():.3g}")
        return
    np.testing.assert_allclose(got, want, rtol=spec["rtol"], atol=spec["atol"], err_msg=what)
