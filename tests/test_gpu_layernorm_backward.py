"""GPU parity of credit_layernorm_bwd_f32 / _bf16 (the reference workload
layernorm_backward, dsmem_eval/workloads.py:53-61) against the float64 oracle.

Tolerances: fp32 dx within rtol 1e-5 / atol 1e-6 (tighter than the
reference's own 2e-2, workloads.py:164-165); bf16 dx within 1e-2 / 1e-2.
Inputs: the reference's Python ranges (x, dy ~ U(-1, 1), gamma ~ U(0.75,
1.25); workloads.py:45-50) and the CUDA binary's hash-LCG closed forms
(src/workloads/layernorm_backward.cu:253-272, restated by
oracle.reference.layernorm_backward_init)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

EPS = 1.0e-5
FP32 = dict(rtol=1e-5, atol=1e-6)
BF16 = dict(rtol=1e-2, atol=1e-2)
STAGED_COLS = {torch.float32: 32768, torch.bfloat16: 32768}


def run(x, dy, gamma, variant, split, gpu):
    ins = [t.to(gpu) for t in (x, dy, gamma)]
    dx = torch.full_like(ins[0], float("nan"))
    hip_lib.layernorm_backward(*ins, dx, EPS, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return dx.float().cpu().numpy()


def expect(x, dy, gamma):
    return ref.layernorm_backward(x.float().numpy(), dy.float().numpy(), gamma.float().numpy(),
                                  EPS)


VARIANTS = [("auto", 0), ("staged", 0), ("read", 0), ("split", 2), ("split", 3), ("split", 8)]
SHAPES = [(16, 4096), (5, 16), (3, 65536), (9, 4104), (33, 1024)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("variant,split", VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_layernorm_backward_shapes(gpu, dtype, variant, split, shape):
    print(f"layernorm_backward {dtype} {variant} P={split} shape={shape}", flush=True)
    spec = WORKLOADS["layernorm_backward" if dtype == torch.float32 else "layernorm_backward_bf16"]
    x, dy, gamma = spec.make_inputs(*shape, seed=81)
    tol = FP32 if dtype == torch.float32 else BF16
    if variant == "staged" and shape[1] > STAGED_COLS[dtype]:
        with pytest.raises(hip_lib.CreditError) as err:
            run(x, dy, gamma, variant, split, gpu)
        assert err.value.status == -4
        return
    np.testing.assert_allclose(run(x, dy, gamma, variant, split, gpu), expect(x, dy, gamma), **tol)


@pytest.mark.parametrize("shape", [(5, 1003), (3, 3), (2, 70001)])
def test_layernorm_backward_ragged_rows_take_read(gpu, shape):
    x, dy, gamma = WORKLOADS["layernorm_backward"].make_inputs(*shape, seed=2)
    np.testing.assert_allclose(run(x, dy, gamma, "auto", 0, gpu), expect(x, dy, gamma), **FP32)
    with pytest.raises(hip_lib.CreditError) as err:
        run(x, dy, gamma, "split", 2, gpu)
    assert err.value.status == -4


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0), ("split", 4)])
def test_layernorm_backward_offset_and_constant_rows(gpu, variant, split):
    """A large common offset (the case one-pass E[x^2] - mean^2 gets wrong)
    and a constant row (variance 0: dx = (g - mean g) / sqrt(eps))."""
    x, dy, gamma = WORKLOADS["layernorm_backward"].make_inputs(4, 8192, seed=12)
    x[0] += 1000.0
    x[1] = 0.25
    got = run(x, dy, gamma, variant, split, gpu)
    np.testing.assert_allclose(got[1:], expect(x, dy, gamma)[1:], **FP32)
    # Row 0: float32 x has ulp 6e-5 at 1000, so the statistics the kernel
    # sees are those of the rounded inputs; compare to the oracle on them.
    np.testing.assert_allclose(got[0], expect(x, dy, gamma)[0], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("n", [4096, 16384, 65536])
def test_layernorm_backward_reference_binary_inputs(gpu, n):
    """The inputs the reference CUDA binary generates on the device
    (hash-LCG closed forms), at its row count capped as quick mode does."""
    xs, dys, gs = ref.layernorm_backward_init(128, n)
    x, dy, gamma = (torch.from_numpy(a) for a in (xs, dys, gs))
    e = expect(x, dy, gamma)
    for variant, split in [("auto", 0), ("read", 0), ("split", 2), ("split", 8)]:
        np.testing.assert_allclose(run(x, dy, gamma, variant, split, gpu), e, **FP32)


def test_layernorm_backward_full_reference_shape(gpu):
    """rows = 2048 (workloads.py:159), the widest N = 65536."""
    x, dy, gamma = WORKLOADS["layernorm_backward"].make_inputs()
    e = expect(x, dy, gamma)
    for variant, split in [("auto", 0), ("split", 4), ("read", 0)]:
        np.testing.assert_allclose(run(x, dy, gamma, variant, split, gpu), e, **FP32)


@pytest.mark.parametrize("variant,split,shape", [
    ("auto", 0, (2048, 65536)),    # the reference shape: the group pipeline, 8 members
    ("split", 16, (2048, 65536)),  # 16 members of 512 vectors (the 256-lane kernel)
    ("split", 2, (2048, 65536)),   # slices too wide for the group pipeline: slice kernel
    ("auto", 0, (40, 131072)),     # 16 members of 1024 vectors
    ("split", 5, (64, 40960)),     # a non-power-of-two group
    ("split", 4, (1, 32768)),      # one row: every group but one is padding
])
def test_layernorm_backward_bf16_group_pipeline(gpu, variant, split, shape):
    """bf16 rows wider than one workgroup take the group pipeline (one
    exchange of four shifted sums per row), against the float64 oracle."""
    print(f"layernorm_backward bf16 {variant} P={split} shape={shape}", flush=True)
    x, dy, gamma = WORKLOADS["layernorm_backward_bf16"].make_inputs(*shape, seed=17)
    np.testing.assert_allclose(run(x, dy, gamma, variant, split, gpu), expect(x, dy, gamma), **BF16)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 8), ("split", 3)])
def test_layernorm_backward_bf16_offset_spike_and_constant_rows(gpu, variant, split):
    """Rows the shifted sums must survive: a large common offset, a spike as
    the row's first element x0 (the shift point far from the mean), a
    constant row (variance 0), at 65536 columns."""
    x, dy, gamma = WORKLOADS["layernorm_backward_bf16"].make_inputs(6, 65536, seed=23)
    x = x.float()
    x[0] += 1000.0
    x[1, 0] = 300.0
    x[2] = 0.25
    x[3, 0] = -500.0
    x[3, 1:] *= 4.0
    x = x.to(torch.bfloat16)
    np.testing.assert_allclose(run(x, dy, gamma, variant, split, gpu), expect(x, dy, gamma), **BF16)
