"""GPU parity of credit_rowwise_quant_f32 against the oracle, the reference
workload rowwise_quant (dsmem_eval/workloads.py:150-154; kernels
src/workloads/rowwise_quant.cu:260-363).

The bar is bit-exact for both outputs: q is integer, and the scale is one
fp32 division of the exact row maximum, so it has one correct value (the
reference asks only 1e-6 of the scale, dsmem_eval/workloads.py:209-210, and
int8-exact q, rowwise_quant.cu:560,569)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

SPEC = WORKLOADS["rowwise_quant"]


def quant(x, variant, split, gpu):
    xs = x.to(gpu)
    q = torch.full(x.shape, -128, dtype=torch.int8, device=gpu)
    scale = torch.full((x.shape[0],), float("nan"), device=gpu)
    hip_lib.rowwise_quant(xs, q, scale, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return q.cpu().numpy(), scale.cpu().numpy()


def check(x, q, scale):
    eq, es = ref.rowwise_quant(x.numpy())
    assert np.array_equal(scale, es), np.flatnonzero(scale != es)[:8]
    bad = np.argwhere(q != eq)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[:4].tolist()}"


def hash_lcg_inputs(rows, cols):
    """The CUDA workload's deterministic input (rowwise_quant.cu:246-258):
    two 64-bit LCG steps of the flat index, shifted right 16 and truncated
    to 32 bits; a grid of 1/2048 steps in [-1, 1) plus a perturbation below
    2.6e-5.  Every step is exact in fp32 except the last two roundings,
    which numpy's float32 arithmetic performs the same way."""
    idx = np.arange(rows * cols, dtype=np.uint64)
    a = ((idx * np.uint64(1103515245) + np.uint64(12345)) >> np.uint64(16)) & np.uint64(0xFFFFFFFF)
    b = ((idx * np.uint64(1664525) + np.uint64(1013904223)) >> np.uint64(16)) & np.uint64(0xFFFFFFFF)
    base = (a & np.uint64(4095)).astype(np.float32) * np.float32(1.0 / 2048.0) - np.float32(1.0)
    tiny = (b & np.uint64(255)).astype(np.float32) * np.float32(1.0e-7)
    return torch.from_numpy((base + tiny).astype(np.float32).reshape(rows, cols))


def tie_rows(rows, cols, seed):
    """Rows whose elements sit next to half-integer codes, (j + 0.5) * m / 127
    with the row maximum m last: the last bit of 1/m decides their rounding."""
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(rows, 1, generator=g) * 3.5 + 0.5
    j = torch.arange(cols - 1, dtype=torch.float32)[None, :] % 127
    sign = torch.where(torch.rand(rows, cols - 1, generator=g) < 0.5, -1.0, 1.0)
    return torch.cat([sign * (j + 0.5) * m / 127.0, m], dim=1).contiguous()


VARIANTS = [("auto", 0), ("staged", 0), ("read", 0), ("split", 2), ("split", 3), ("split", 8)]
SHAPES = [(16, 4096), (5, 12), (3, 65536), (9, 4100), (33, 1024), (2, 4)]


@pytest.mark.parametrize("variant,split", VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_quant_shapes(gpu, variant, split, shape):
    print(f"rowwise_quant {variant} P={split} shape={shape}", flush=True)
    (x,) = SPEC.make_inputs(*shape, seed=61)
    check(x, *quant(x, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0)])
@pytest.mark.parametrize("shape", [(7, 4097), (3, 1), (4, 30)])
def test_quant_unaligned_widths(gpu, variant, split, shape):
    """cols % 4 != 0: the scalar READ path."""
    print(f"rowwise_quant {variant} shape={shape}", flush=True)
    (x,) = SPEC.make_inputs(*shape, seed=62)
    check(x, *quant(x, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 4), ("split", 16), ("read", 0)])
def test_quant_wide_rows(gpu, variant, split):
    (x,) = SPEC.make_inputs(6, 262144, seed=63)
    check(x, *quant(x, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("staged", 0), ("split", 4), ("read", 0)])
def test_quant_ties_and_special_rows(gpu, variant, split):
    """Tie-adjacent rows, an all-zero row (scale 0, q 0), a row whose
    maximum is negative, and a row with a single non-zero element."""
    print(f"rowwise_quant ties {variant} P={split}", flush=True)
    x = tie_rows(64, 8192, seed=64)
    x[3] = 0.0
    x[5] = -x[5].abs()
    x[9] = 0.0
    x[9, 4321] = -3.0e-30
    check(x, *quant(x, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 2), ("read", 0)])
def test_quant_hash_lcg_inputs(gpu, variant, split):
    """The CUDA workload's own input generator at one of its widths."""
    x = hash_lcg_inputs(32, 16384)
    check(x, *quant(x, variant, split, gpu))


def test_quant_zero_rows(gpu):
    x = torch.empty(0, 64)
    q, scale = quant(x, "auto", 0, gpu)
    assert q.shape == (0, 64) and scale.shape == (0,)


def test_quant_rejects_bad_split(gpu):
    (x,) = SPEC.make_inputs(2, 131072, seed=65)
    xs = x.to(gpu)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(2, device=gpu)
    with pytest.raises(hip_lib.CreditError):
        hip_lib.rowwise_quant(xs, q, s, hip_lib.make_cfg("staged", 0))
    with pytest.raises(hip_lib.CreditError):
        hip_lib.rowwise_quant(xs, q, s, hip_lib.make_cfg("split", 1))


@pytest.mark.parametrize("split", [2, 8])
def test_quant_back_to_back(gpu, split):
    """Six split launches queued with no host synchronisation, each group
    taking several rows; the last result is checked."""
    (x,) = SPEC.make_inputs(2048, 16384, seed=66)
    xs = x.to(gpu)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], device=gpu)
    cfg = hip_lib.make_cfg("split", split)
    print(f"rowwise_quant back to back P={split}", flush=True)
    for _ in range(6):
        hip_lib.rowwise_quant(xs, q, s, cfg)
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    check(x, q.cpu().numpy(), s.cpu().numpy())


def test_quant_full_shape_properties(gpu):
    """The bench shape (4096 x 65536): every code in [-127, 127], each row's
    largest |code| is 127 where its maximum is non-zero, the scale is
    max|x| / 127, and dequantisation stays within half a step."""
    (x,) = SPEC.make_inputs()
    xs = x.to(gpu)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], device=gpu)
    hip_lib.rowwise_quant(xs, q, s, hip_lib.make_cfg())
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    assert int(q.min()) >= -127
    amax = xs.abs().amax(dim=1)
    assert torch.equal(s, amax / torch.tensor(127.0, device=gpu))
    assert torch.equal(q.abs().amax(dim=1).int(), torch.full_like(s, 127).int())
    err = (q.float() * s[:, None] - xs).abs() - s[:, None] * 0.5
    assert float(err.max()) <= 1e-6
    # A slice of rows against the oracle, bit-exact.
    check(x[:64], q[:64].cpu().numpy(), s[:64].cpu().numpy())
