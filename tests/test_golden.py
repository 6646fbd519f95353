"""The CPU oracle (oracle/reference.py) against the golden fixtures, whose
expected outputs tests/golden/make_golden.py computed with torch's own
float64 routines and autograd, independently of the oracle.

Where both sides are float64 evaluations of the same inputs the oracle must
agree to 1e-9; where a side rounds (the fp32 rstd input of the RMSNorm
backward, bf16 activations of the FFN, the fp32 LARS update, the weighted
variance formula's dropped O(eps) term) it must meet the fixture's own check,
the bar the GPU results are held to."""
import numpy as np
import pytest

from oracle import reference as ref
from tests.golden import fixtures

TIGHT = {"check": "allclose", "rtol": 1e-9, "atol": 1e-12}


def f32(t):
    return t.float().numpy()


def oracle_outputs(name, ins):
    """(oracle outputs, per-output checks: None = the fixture's own)."""
    a = [f32(t) for t in ins]
    if name == "row_sum_max":
        return ref.row_sum_max(a[0]), [TIGHT, None]
    if name == "layernorm_fwd":
        return ref.layernorm_fwd(a[0], a[1], a[2], 1e-5), [TIGHT, TIGHT, TIGHT]
    if name == "rmsnorm_fwd":
        return ref.rmsnorm_fwd(a[0], a[1], 1e-6), [TIGHT, TIGHT]
    if name == "rmsnorm_bwd":
        return ref.rmsnorm_bwd(a[0], a[1], a[2], a[3]), [None, None]
    if name == "rmsnorm_fwd_bwd":
        # float64 rstd: the fixture is float64 autograd end to end
        return ref.rmsnorm_fwd_bwd(a[0], a[1], a[2], 1e-6, rstd_fp32=False), [TIGHT] * 4
    if name == "softmax_fwd":
        return ref.softmax_fwd(a[0]), [TIGHT, None, TIGHT]
    if name == "softmax_bwd":
        return (ref.softmax_bwd(a[0], a[1]),), [TIGHT]
    if name == "softmax_logits_backward":
        return (ref.softmax_logits_backward(a[0], a[1]),), [TIGHT]
    if name in ("layernorm_backward", "layernorm_backward_bf16"):
        return (ref.layernorm_backward(a[0], a[1], a[2], 1e-5),), [TIGHT]
    if name == "rowwise_quant":
        return ref.rowwise_quant(a[0]), [None, None]
    if name == "lars_momentum":
        w, u = ref.lars_momentum(a[0], a[1], a[2])
        return (w, u), [TIGHT, {"check": "allclose", "rtol": 1e-6, "atol": 1e-7}]
    if name == "weighted_var_backward":
        return (ref.weighted_var_backward(a[0], a[1], a[2]),), [
            {"check": "allclose", "rtol": 1e-6, "atol": 1e-8}]
    if name == "pearson_backward":
        return ref.pearson_backward(a[0], a[1], a[2]), [TIGHT, TIGHT]
    if name == "ffn":
        # the fixture keeps RMSNorm(x) unrounded; the oracle rounds it to bf16
        return (ref.ffn_rmsnorm_gelu(a[0], a[1].T, a[2].T, 1e-6),), [None]
    raise KeyError(name)


@pytest.mark.parametrize("case", fixtures.cases())
def test_oracle_matches_golden(case):
    meta, ins, expected = fixtures.load(case)
    outs, checks = oracle_outputs(meta["workload"], ins)
    assert len(outs) == len(expected)
    for i, (got, want) in enumerate(zip(outs, expected)):
        spec = checks[i] if checks[i] is not None else meta["checks"][i]
        fixtures.check(got, want, spec, f"{case} output {i}")


def test_golden_set_covers_every_launcher():
    from credit_amd.hip_lib import HIP_LAUNCHERS

    covered = {fixtures.load(c)[0]["workload"] for c in fixtures.cases()}
    # ffn_baseline_layout runs the ffn fixture with its weights transposed
    # to [in, out] (tests/test_gpu_golden.py).
    # The FFN backward forms are held to the float64 oracle on the GPU
    # (tests/test_gpu_ffn_backward.py), not by fixtures.
    assert covered == set(HIP_LAUNCHERS) - {"ffn_backward", "ffn_backward_saved",
                                             "ffn_backward_baseline_layout",
                                             "ffn_baseline_layout"}


def test_golden_fixtures_catch_a_planted_mistake():
    """A LayerNorm backward without its mean(dyg * xhat) term, planted in a
    copy of the oracle's arithmetic, fails the fixture."""
    meta, ins, expected = fixtures.load("layernorm_backward_3x4096")
    x, dy, g = (f32(t).astype(np.float64) for t in ins)
    xmu = x - x.mean(-1, keepdims=True)
    inv = 1 / np.sqrt((xmu * xmu).mean(-1, keepdims=True) + 1e-5)
    dyg = dy * g
    wrong = (dyg - dyg.mean(-1, keepdims=True)) * inv
    with pytest.raises(AssertionError):
        fixtures.check(wrong, expected[0], meta["checks"][0], "planted")


def test_rowmax_check_scales_atol_per_row():
    want = np.array([[1e-5, 2e-5], [1.0, 2.0]])
    spec = {"check": "rowmax", "rtol": 1e-5, "atol": 1e-6}
    fixtures.check(want + np.array([[1e-11, 0], [1e-6, 0]]), want, spec, "within")
    with pytest.raises(AssertionError):
        fixtures.check(want + np.array([[1e-9, 0], [0, 0]]), want, spec, "outside")
