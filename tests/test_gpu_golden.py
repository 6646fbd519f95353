"""The HIP library against the golden fixtures (tests/golden/*.npz), through
the launcher table, for every variant each fixture lists.  The fixtures'
expected outputs are torch float64 routines / autograd (make_golden.py);
each output is held to the check stored with it: fp32 rtol 1e-5 / atol 1e-6,
bf16 rtol 1e-2 / atol 1e-2, maxima, int8 codes, scales and the LARS update
bit-exact."""
import pytest
import torch

from credit_amd import hip_lib
from tests.golden import fixtures

pytestmark = pytest.mark.gpu

RUNS = [(c, v, p) for c in fixtures.cases() for v, p in fixtures.load(c)[0]["variants"]]


@pytest.mark.parametrize("case,variant,split", RUNS)
def test_hip_matches_golden(gpu, case, variant, split):
    print(f"golden {case} {variant} P={split}", flush=True)
    meta, ins, expected = fixtures.load(case)
    name = meta["workload"]
    gins = tuple(t.to(gpu) for t in ins)
    outs = hip_lib.allocate_outputs(name, gins)
    for o in outs:
        if o.is_floating_point():
            o.fill_(float("nan"))
    hip_lib.HIP_LAUNCHERS[name](gins, outs, hip_lib.LaunchConfig(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    for i, (o, want) in enumerate(zip(outs, expected)):
        got = o.float().cpu().numpy() if o.is_floating_point() else o.cpu().numpy()
        fixtures.check(got, want, meta["checks"][i], f"{case} {variant} output {i}")


@pytest.mark.parametrize("case,variant,split", [("rmsnorm_bwd_3x8192", "split", 2),
                                                ("softmax_fwd_3x5000", "auto", 0),
                                                ("layernorm_fwd_9x4096", "staged", 0)])
def test_bound_launcher_matches_golden(gpu, case, variant, split):
    """hip_lib.bind (the argument-converted-once form bench.py times) runs the
    same library calls: each of two calls meets the fixture, and a variant
    the library refuses raises at call time."""
    meta, ins, expected = fixtures.load(case)
    name = meta["workload"]
    gins = tuple(t.to(gpu) for t in ins)
    outs = hip_lib.allocate_outputs(name, gins)
    call = hip_lib.bind(name, gins, outs, hip_lib.LaunchConfig(variant, split))
    for _ in range(2):
        for o in outs:
            if o.is_floating_point():
                o.fill_(float("nan"))
        call()
        torch.cuda.synchronize()
        for i, (o, want) in enumerate(zip(outs, expected)):
            got = o.float().cpu().numpy()
            fixtures.check(got, want, meta["checks"][i], f"bound {case} output {i}")
    bad = hip_lib.bind(name, gins, outs, hip_lib.LaunchConfig("split", 1 << 20))
    with pytest.raises(hip_lib.CreditError):
        bad()


def test_ffn_in_out_layout_matches_golden(gpu):
    """The ffn fixture (weights in the nn.Linear layout) through the [in, out]
    weight entry point, its weights transposed on the host."""
    meta, ins, expected = fixtures.load("ffn_128x128x256")
    x, w1l, w2l = ins
    gins = (x.to(gpu), w1l.t().contiguous().to(gpu), w2l.t().contiguous().to(gpu))
    (out,) = hip_lib.allocate_outputs("ffn_baseline_layout", gins)
    out.fill_(float("nan"))
    hip_lib.HIP_LAUNCHERS["ffn_baseline_layout"](gins, (out,))
    torch.cuda.synchronize()
    fixtures.check(out.float().cpu().numpy(), expected[0], meta["checks"][0], "ffn in_out")
