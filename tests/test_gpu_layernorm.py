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
    """Shapes the staged layout does not cover fall back to the READ kernel
    under AUTO and are rejected under an explicit STAGED request."""
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
