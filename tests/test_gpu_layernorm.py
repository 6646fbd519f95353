"""GPU parity of credit_layernorm_fwd_bf16 (C2) against the CPU oracle.

Tolerances: y (bf16) within rtol 1e-2 / atol 1e-2; mean and rstd (fp32)
within rtol 1e-5 / atol 1e-6 of the float64 statistics."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

SPEC = WORKLOADS["layernorm_fwd"]
EPS = 1.0e-5


def run(x, g, b, variant, gpu):
    ins = tuple(t.to(gpu) for t in (x, g, b))
    y, mean, rstd = hip_lib.allocate_outputs("layernorm_fwd", ins)
    hip_lib.layernorm_fwd(*ins, y, mean, rstd, EPS, hip_lib.make_cfg(variant))
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), mean.cpu().numpy(), rstd.cpu().numpy()


def check(x, g, b, y, mean, rstd):
    ey, em, er = ref.layernorm_fwd(x.float().numpy(), g.float().numpy(), b.float().numpy(), EPS)
    np.testing.assert_allclose(mean, em, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd, er, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(y, ey, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("variant", ["auto", "staged", "read"])
@pytest.mark.parametrize("shape", [(16, 4096), (7, 8), (3, 2048), (5, 24576), (2, 65536), (33, 32768)])
def test_layernorm_fwd_shapes(gpu, variant, shape):
    print(f"layernorm_fwd {variant} shape={shape}", flush=True)
    x, g, b = SPEC.make_inputs(*shape, seed=21)
    check(x, g, b, *run(x, g, b, variant, gpu))


@pytest.mark.parametrize("shape", [(5, 1004), (3, 3), (2, 140000), (2, 131072)])
def test_layernorm_fwd_read_only_shapes(gpu, shape):
    """Shapes the staged layout does not cover (cols % 8 != 0: the READ
    kernel's element loads; rows wider than 65536 columns: SPLIT) run under
    AUTO and are rejected under an explicit STAGED request."""
    x, g, b = SPEC.make_inputs(*shape, seed=4)
    check(x, g, b, *run(x, g, b, "auto", gpu))
    with pytest.raises(hip_lib.CreditError) as err:
        run(x, g, b, "staged", gpu)
    assert err.value.status == -4


def test_layernorm_fwd_constant_rows(gpu):
    x, g, b = SPEC.make_inputs(4, 4096, seed=1)
    x[0, :] = 1.5
    x[1, :] = 0.0
    y, mean, rstd = run(x, g, b, "staged", gpu)
    assert mean[0] == 1.5 and mean[1] == 0.0
    np.testing.assert_allclose(rstd[:2], 1 / np.sqrt(EPS), rtol=1e-6)
    np.testing.assert_allclose(y[0], b.float().numpy(), atol=1e-6)
    check(x, g, b, y, mean, rstd)


@pytest.mark.parametrize("variant", ["auto", "read"])
def test_layernorm_fwd_full_config(gpu, variant):
    """BASELINE C2: 2048 x 32768 bf16, N(0,1); gamma N(1,.02), beta N(0,.02)."""
    x, g, b = SPEC.make_inputs()
    check(x, g, b, *run(x, g, b, variant, gpu))


@pytest.mark.parametrize("shape", [(512, 32768), (773, 32768), (600, 24576), (1030, 16392),
                                   (2049, 20000)])
def test_layernorm_fwd_pipeline_rows(gpu, shape):
    """AUTO's persistent pipeline (2049..4096 vectors per row, at least two
    rows per CU): row counts that end the three-row rotation at each of its
    steps, rows shorter than the 4096-vector layout, and the same rows
    through the one-row-per-workgroup STAGED kernel, which must agree with it
    up to the fp32 summation order."""
    print(f"layernorm_fwd pipeline shape={shape}", flush=True)
    x, g, b = SPEC.make_inputs(*shape, seed=37)
    x[5, :] = 2.25  # a constant row: var = 0, y = beta
    y, mean, rstd = run(x, g, b, "auto", gpu)
    check(x, g, b, y, mean, rstd)
    assert mean[5] == 2.25
    np.testing.assert_allclose(y[5], b.float().numpy(), atol=1e-6)
    sy, smean, srstd = run(x, g, b, "staged", gpu)
    np.testing.assert_allclose(mean, smean, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(rstd, srstd, rtol=1e-6)
    np.testing.assert_allclose(y, sy, rtol=1e-2, atol=1e-2)  # bf16 rounding flips only


def test_layernorm_fwd_pipeline_back_to_back(gpu):
    """Calls queued without synchronisation on one stream, each checked."""
    x, g, b = SPEC.make_inputs(700, 32768, seed=3)
    ins = tuple(t.to(gpu) for t in (x, g, b))
    outs = [hip_lib.allocate_outputs("layernorm_fwd", ins) for _ in range(3)]
    for o in outs:
        hip_lib.layernorm_fwd(*ins, *o, EPS, hip_lib.make_cfg("auto"))
    torch.cuda.synchronize()
    first = [t.cpu() for t in outs[0]]
    for o in outs[1:]:
        for a, b_ in zip(first, o):
            assert torch.equal(a, b_.cpu())
    check(x, g, b, *(t.float().numpy() for t in first))


@pytest.mark.parametrize("shape", [(600, 32768), (520, 24576)])
def test_layernorm_fwd_offset_rows_take_the_two_pass_statistics(gpu, shape):
    """Rows whose mean is large against their spread (mean^2 > var/4) leave
    the one-pass sums for the second pass over squared deviations; rows with
    a small offset stay on the one-pass path.  Both agree with the float64
    two-pass oracle at fp32 tolerance, in the pipeline and in STAGED."""
    x, g, b = SPEC.make_inputs(*shape, seed=41)
    xf = x.float()
    xf[0::4] = xf[0::4] * 0.01 + 300.0  # mean^2 / var ~ 1e9: two-pass
    xf[1::4] = xf[1::4] + 0.4           # mean^2 / var = 0.16: one-pass
    xf[2::4] = xf[2::4] * 1e-3 - 5e-4   # small values, small offset
    x = xf.bfloat16()
    for variant in ("auto", "staged"):
        print(f"layernorm_fwd offset rows {variant} shape={shape}", flush=True)
        check(x, g, b, *run(x, g, b, variant, gpu))


@pytest.mark.parametrize("shape,variant,split", [((2, 140000), "auto", 0), ((256, 262144), "auto", 0),
                                                 ((5, 131072), "split", 4), ((5, 131072), "split", 5),
                                                 ((9, 65536), "split", 8), ((300, 100000), "auto", 0),
                                                 ((3, 140000), "read", 0)])
def test_layernorm_fwd_wide_rows(gpu, shape, variant, split):
    """Rows wider than one workgroup holds: the SPLIT kernel (members
    exchanging (sum, sum of squares); ragged last members at 140000 and
    100000 columns; more rows than resident groups at 300 x 100000) and the
    vectorised READ kernel, against the float64 two-pass oracle."""
    print(f"layernorm_fwd wide {variant} P={split} shape={shape}", flush=True)
    x, g, b = SPEC.make_inputs(*shape, seed=shape[0] + split)
    y, mean, rstd = run_split(x, g, b, variant, split, gpu)
    check(x, g, b, y, mean, rstd)


def test_layernorm_fwd_split_offset_and_constant_rows(gpu):
    """The SPLIT kernel's second exchange stage (squared deviations) for
    rows with a large offset, and constant rows, mixed with one-pass rows."""
    x, g, b = SPEC.make_inputs(40, 139264, seed=5)
    xf = x.float()
    xf[0::3] = xf[0::3] * 0.01 + 300.0
    xf[1] = 2.25
    x = xf.bfloat16()
    for variant, split in (("auto", 0), ("split", 5)):
        print(f"layernorm_fwd offset rows {variant} P={split}", flush=True)
        y, mean, rstd = run_split(x, g, b, variant, split, gpu)
        check(x, g, b, y, mean, rstd)
        assert mean[1] == 2.25
        np.testing.assert_allclose(y[1], b.float().numpy(), atol=1e-6)


def test_layernorm_fwd_split_rejections(gpu):
    x, g, b = SPEC.make_inputs(2, 65536, seed=1)
    with pytest.raises(hip_lib.CreditError) as err:
        run_split(x, g, b, "split", 33, gpu)  # 33 members exchange 66 partials
    assert err.value.status == -4
    x, g, b = SPEC.make_inputs(2, 131072, seed=1)
    with pytest.raises(hip_lib.CreditError) as err:
        run_split(x, g, b, "split", 2, gpu)  # 8192 vectors per member: at most 4096
    assert err.value.status == -4
    x, g, b = SPEC.make_inputs(2, 65544 + 4, seed=1)  # cols % 8 != 0
    with pytest.raises(hip_lib.CreditError) as err:
        run_split(x, g, b, "split", 2, gpu)
    assert err.value.status == -4


def run_split(x, g, b, variant, split, gpu):
    ins = tuple(t.to(gpu) for t in (x, g, b))
    y, mean, rstd = hip_lib.allocate_outputs("layernorm_fwd", ins)
    hip_lib.layernorm_fwd(*ins, y, mean, rstd, EPS, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return y.float().cpu().numpy(), mean.cpu().numpy(), rstd.cpu().numpy()
