"""GPU parity of credit_row_sum_max_f32 (C1) against the CPU oracle.

Tolerances: sum within rtol 1e-5 / atol 1e-6 of the float64 sum; max
bit-exact (including NaN rows)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

SPEC = WORKLOADS["row_sum_max"]
VARIANTS = [("auto", 0), ("read", 0), ("split", 2), ("split", 4), ("split", 7), ("split", 16)]


def run(x_cpu, variant, split, gpu, offset=0):
    rows, cols = x_cpu.shape
    if offset:
        flat = torch.empty(rows * cols + offset, dtype=torch.float32, device=gpu)
        x = flat[offset:].view(rows, cols)
        x.copy_(x_cpu)
    else:
        x = x_cpu.to(gpu)
    s = torch.full((rows,), float("nan"), device=gpu)
    m = torch.full((rows,), float("nan"), device=gpu)
    hip_lib.row_sum_max(x, s, m, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return s.cpu().numpy(), m.cpu().numpy()


def check(x_cpu, s, m):
    es, em = ref.row_sum_max(x_cpu.numpy())
    np.testing.assert_allclose(s, es, rtol=1e-5, atol=1e-6)
    em32 = em.astype(np.float32)
    assert np.array_equal(np.isnan(m), np.isnan(em32))
    assert np.array_equal(m[~np.isnan(m)], em32[~np.isnan(em32)])


@pytest.mark.parametrize("variant,split", VARIANTS)
@pytest.mark.parametrize("shape", [(64, 4100), (5, 3), (3, 1), (17, 65536), (8, 4097), (1, 262147)])
def test_row_sum_max_shapes(gpu, variant, split, shape):
    print(f"row_sum_max {variant} P={split} shape={shape}", flush=True)
    (x,) = SPEC.make_inputs(*shape, seed=11)
    s, m = run(x, variant, split, gpu)
    check(x, s, m)


@pytest.mark.parametrize("variant,split", VARIANTS)
def test_row_sum_max_misaligned_rows(gpu, variant, split):
    (x,) = SPEC.make_inputs(9, 1030, seed=3)
    s, m = run(x, variant, split, gpu, offset=1)
    check(x, s, m)


@pytest.mark.parametrize("variant,split", [("read", 0), ("split", 4)])
def test_row_sum_max_special_values(gpu, variant, split):
    (x,) = SPEC.make_inputs(6, 5000, seed=5)
    x[0, 1234] = float("nan")
    x[1, 7] = float("inf")
    x[2, :] = -float("inf")
    x[3, :] = 0.0
    x[4, 4999] = 1.0e30
    x[5, :] = -2.5
    s, m = run(x, variant, split, gpu)
    es, em = ref.row_sum_max(x.numpy())
    assert np.isnan(m[0]) and np.isnan(s[0])
    assert m[1] == np.inf and s[1] == np.inf
    assert m[2] == -np.inf and s[2] == -np.inf
    assert m[3] == 0.0 and s[3] == 0.0
    assert m[4] == np.float32(1.0e30)
    assert m[5] == -2.5 and s[5] == -12500.0


def test_row_sum_max_split_repeats_and_shrinks(gpu):
    """The arrival counters reset themselves: repeated split calls, and a call
    with fewer rows after a larger one, stay correct."""
    for rows, cols in [(300, 8192), (300, 8192), (40, 20000), (300, 8192)]:
        (x,) = SPEC.make_inputs(rows, cols, seed=rows + cols)
        s, m = run(x, "split", 4, gpu)
        check(x, s, m)


def test_row_sum_max_caller_workspace(gpu):
    (x,) = SPEC.make_inputs(128, 16384, seed=9)
    nbytes = hip_lib.workspace_bytes("row_sum_max", 128, 16384, "split", 8)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    xs = x.to(gpu)
    s = torch.empty(128, device=gpu)
    m = torch.empty(128, device=gpu)
    for _ in range(3):
        hip_lib.row_sum_max(xs, s, m, hip_lib.make_cfg("split", 8, workspace=ws))
        torch.cuda.synchronize()
        check(x, s.cpu().numpy(), m.cpu().numpy())
    small = torch.zeros(64, dtype=torch.uint8, device=gpu)
    with pytest.raises(hip_lib.CreditError) as err:
        hip_lib.row_sum_max(xs, s, m, hip_lib.make_cfg("split", 8, workspace=small))
    assert err.value.status == -5


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0), ("split", 2), ("split", 4)])
def test_row_sum_max_full_config(gpu, variant, split):
    """BASELINE C1: 1024 x 65536 fp32, U(-1,1), seed 0."""
    (x,) = SPEC.make_inputs()
    s, m = run(x, variant, split, gpu)
    check(x, s, m)
