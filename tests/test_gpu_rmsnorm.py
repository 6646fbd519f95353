"""GPU parity of credit_rmsnorm_fwd_bf16 / credit_rmsnorm_bwd_bf16 (C3)
against the float64 CPU oracle.

Tolerances: bf16 outputs (y, dx) within rtol 1e-2 /
atol 1e-2; fp32 outputs (rstd, dweight) within rtol 1e-5 / atol 1e-6.  The
backward takes rstd as an input, so the oracle is given the same fp32 rstd
the kernel gets (the forward oracle's rstd rounded to fp32)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

SPEC = WORKLOADS["rmsnorm_fwd"]
EPS = 1.0e-6
BF16 = dict(rtol=1e-2, atol=1e-2)
FP32 = dict(rtol=1e-5, atol=1e-6)


def fwd(x, w, variant, split, gpu):
    xs, ws_ = x.to(gpu), w.to(gpu)
    y = torch.empty_like(xs)
    rstd = torch.full((x.shape[0],), float("nan"), device=gpu)
    hip_lib.rmsnorm_fwd(xs, ws_, y, rstd, EPS, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return y.float().cpu().numpy(), rstd.cpu().numpy()


def check_fwd(x, w, y, rstd):
    ey, er = ref.rmsnorm_fwd(x.float().numpy(), w.float().numpy(), EPS)
    np.testing.assert_allclose(rstd, er, **FP32)
    np.testing.assert_allclose(y, ey, **BF16)


def bwd(x, w, dy, rstd32, variant, split, gpu):
    ins = [t.to(gpu) for t in (x, w, dy)]
    r = torch.from_numpy(rstd32).to(gpu)
    dx = torch.empty_like(ins[0])
    dw = torch.full((x.shape[1],), float("nan"), device=gpu)
    hip_lib.rmsnorm_bwd(*ins, r, dx, dw, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return dx.float().cpu().numpy(), dw.cpu().numpy()


def oracle_rstd32(x):
    _, er = ref.rmsnorm_fwd(x.float().numpy(), np.ones(x.shape[1]), EPS)
    return er.astype(np.float32)


def check_bwd(x, w, dy, rstd32, dx, dw):
    edx, edw = ref.rmsnorm_bwd(x.float().numpy(), w.float().numpy(), dy.float().numpy(), rstd32)
    np.testing.assert_allclose(dw, edw, **FP32)
    np.testing.assert_allclose(dx, edx, **BF16)


FWD_VARIANTS = [("auto", 0), ("staged", 0), ("read", 0), ("split", 2), ("split", 3), ("split", 8)]


@pytest.mark.parametrize("variant,split", FWD_VARIANTS)
@pytest.mark.parametrize("shape", [(16, 4096), (5, 24), (3, 65536), (9, 8200), (33, 2048)])
def test_rmsnorm_fwd_shapes(gpu, variant, split, shape):
    print(f"rmsnorm_fwd {variant} P={split} shape={shape}", flush=True)
    x, w, _ = SPEC.make_inputs(*shape, seed=31)
    check_fwd(x, w, *fwd(x, w, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 2), ("split", 4), ("read", 0)])
def test_rmsnorm_fwd_wide_rows(gpu, variant, split):
    """Rows wider than one workgroup's registers (C3 width)."""
    x, w, _ = SPEC.make_inputs(4, 131072, seed=7)
    check_fwd(x, w, *fwd(x, w, variant, split, gpu))


@pytest.mark.parametrize("rows,cols,variant,split", [
    (4, 131072, "auto", 0),    # 8 members of 2048 vectors
    (5, 98304, "split", 6),    # 6 members of 2048
    (5, 98304, "split", 7),    # members of 1756 vectors, the last 1752
    (3, 81920, "auto", 0),     # 5 members of 2048
    (7, 65544, "auto", 0),     # 8193 vectors: 5 members of 1639, the last 1637
    (2, 262144, "split", 16),  # 16 members of 2048
    (1, 131072, "auto", 0),
    (300, 98304, "split", 6),  # many rows per group
])
def test_rmsnorm_fwd_group_pipeline(gpu, rows, cols, variant, split):
    """Plans whose members hold 1025-2048 vectors run the forward group
    pipeline (AUTO on rows of 8193-16384 vectors)."""
    print(f"rmsnorm_fwd group {variant} P={split} shape=({rows}, {cols})", flush=True)
    x, w, _ = SPEC.make_inputs(rows, cols, seed=rows + cols)
    check_fwd(x, w, *fwd(x, w, variant, split, gpu))
    # 512 data lanes, the communication wave and the row-ticket wave
    assert hip_lib.last_split_shape()["threads"] == 512 + 128


def test_rmsnorm_fwd_group_zero_constant_and_offset_rows(gpu):
    x, w, _ = SPEC.make_inputs(4, 131072, seed=3)
    x[0, :] = 0.0
    x[1, :] = 2.0
    x[2, :] += 100.0
    y, rstd = fwd(x, w, "auto", 0, gpu)
    np.testing.assert_allclose(rstd[0], 1.0 / np.sqrt(EPS), rtol=1e-6)
    assert np.all(y[0] == 0.0)
    np.testing.assert_allclose(rstd[1], 1.0 / np.sqrt(4.0 + EPS), rtol=1e-6)
    check_fwd(x, w, y, rstd)


def test_rmsnorm_fwd_group_repeats_and_shrinks(gpu):
    for rows in [200, 200, 16, 1, 200]:
        x, w, _ = SPEC.make_inputs(rows, 131072, seed=rows)
        check_fwd(x, w, *fwd(x, w, "auto", 0, gpu))


def test_rmsnorm_fwd_staged_rejects_wide_rows(gpu):
    x, w, _ = SPEC.make_inputs(2, 131072, seed=7)
    with pytest.raises(hip_lib.CreditError) as err:
        fwd(x, w, "staged", 0, gpu)
    assert err.value.status == -4


@pytest.mark.parametrize("shape", [(5, 1004), (3, 3), (2, 1001)])
def test_rmsnorm_fwd_ragged_rows_take_read(gpu, shape):
    x, w, _ = SPEC.make_inputs(*shape, seed=4)
    check_fwd(x, w, *fwd(x, w, "auto", 0, gpu))
    for variant, split in [("staged", 0), ("split", 2)]:
        with pytest.raises(hip_lib.CreditError) as err:
            fwd(x, w, variant, split, gpu)
        assert err.value.status == -4


def test_rmsnorm_fwd_zero_and_constant_rows(gpu):
    x, w, _ = SPEC.make_inputs(3, 4096, seed=2)
    x[0, :] = 0.0
    x[1, :] = 2.0
    y, rstd = fwd(x, w, "split", 4, gpu)
    np.testing.assert_allclose(rstd[0], 1.0 / np.sqrt(EPS), rtol=1e-6)
    assert np.all(y[0] == 0.0)
    np.testing.assert_allclose(rstd[1], 1.0 / np.sqrt(4.0 + EPS), rtol=1e-6)
    check_fwd(x, w, y, rstd)


def test_rmsnorm_fwd_split_repeats_and_shrinks(gpu):
    """Ticket dispenser and group counters return to zero after every call."""
    for rows, cols in [(300, 16384), (300, 16384), (40, 8192), (300, 16384), (1, 16384)]:
        x, w, _ = SPEC.make_inputs(rows, cols, seed=rows + cols)
        check_fwd(x, w, *fwd(x, w, "split", 4, gpu))


def test_rmsnorm_fwd_caller_workspace(gpu):
    x, w, _ = SPEC.make_inputs(64, 16384, seed=9)
    nbytes = hip_lib.workspace_bytes("rmsnorm_fwd", 64, 16384, "split", 4)
    assert nbytes > 0
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    xs, wsb = x.to(gpu), w.to(gpu)
    y = torch.empty_like(xs)
    rstd = torch.empty(64, device=gpu)
    for _ in range(3):
        hip_lib.rmsnorm_fwd(xs, wsb, y, rstd, EPS, hip_lib.make_cfg("split", 4, workspace=ws))
        torch.cuda.synchronize()
        check_fwd(x, w, y.float().cpu().numpy(), rstd.cpu().numpy())
    # Watchdog, exit count and counters back to zero; the tag sequence (header
    # byte 64) advanced by the three launches' stages.
    head = ws[: 256 + 4 * 262144].clone()
    seq = int(head[64:68].cpu().view(torch.int32).item())
    head[64:68] = 0
    assert int(head.count_nonzero()) == 0
    assert seq > 0 and seq % 3 == 0


BWD_VARIANTS = [("auto", 0), ("read", 0), ("split", 2), ("split", 4), ("split", 5)]


@pytest.mark.parametrize("variant,split", BWD_VARIANTS)
@pytest.mark.parametrize("shape", [(16, 4096), (7, 16), (33, 16384), (130, 2048), (3, 24)])
def test_rmsnorm_bwd_shapes(gpu, variant, split, shape):
    print(f"rmsnorm_bwd {variant} P={split} shape={shape}", flush=True)
    x, w, dy = SPEC.make_inputs(*shape, seed=41)
    r = oracle_rstd32(x)
    check_bwd(x, w, dy, r, *bwd(x, w, dy, r, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 16), ("split", 24), ("read", 0)])
def test_rmsnorm_bwd_wide_rows(gpu, variant, split):
    x, w, dy = SPEC.make_inputs(20, 131072, seed=43)
    r = oracle_rstd32(x)
    check_bwd(x, w, dy, r, *bwd(x, w, dy, r, variant, split, gpu))


def test_rmsnorm_bwd_staged_and_short_split_reject_wide_rows(gpu):
    x, w, dy = SPEC.make_inputs(2, 131072, seed=3)
    r = oracle_rstd32(x)
    for variant, split in [("staged", 0), ("split", 2), ("split", 8)]:
        with pytest.raises(hip_lib.CreditError) as err:
            bwd(x, w, dy, r, variant, split, gpu)
        assert err.value.status == -4


def test_rmsnorm_bwd_zero_rows_gives_zero_dweight(gpu):
    backing = torch.zeros(1, 4096, dtype=torch.bfloat16, device=gpu)
    x = backing[:0]  # zero rows, non-null pointer
    w = torch.ones(4096, dtype=torch.bfloat16, device=gpu)
    dx = torch.zeros(1, 4096, dtype=torch.bfloat16, device=gpu)[:0]
    dw = torch.full((4096,), 5.0, device=gpu)
    rstd = torch.ones(1, device=gpu)[:0]
    hip_lib.rmsnorm_bwd(x, w, x, rstd, dx, dw, hip_lib.make_cfg())
    torch.cuda.synchronize()
    assert float(dw.abs().max()) == 0.0


def test_rmsnorm_bwd_is_deterministic(gpu):
    x, w, dy = SPEC.make_inputs(64, 32768, seed=5)
    r = oracle_rstd32(x)
    a = bwd(x, w, dy, r, "split", 4, gpu)
    b = bwd(x, w, dy, r, "split", 4, gpu)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.fixture(scope="module")
def c3_case():
    """BASELINE C3: 1024 x 131072 bf16, x, dy ~ N(0,1), w ~ N(1, 0.02)."""
    x, w, dy = SPEC.make_inputs()
    ey, er = ref.rmsnorm_fwd(x.float().numpy(), w.float().numpy(), EPS)
    r32 = er.astype(np.float32)
    edx, edw = ref.rmsnorm_bwd(x.float().numpy(), w.float().numpy(), dy.float().numpy(), r32)
    return x, w, dy, ey, er, r32, edx, edw


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 2), ("split", 4), ("split", 8),
                                           ("read", 0)])
def test_rmsnorm_fwd_full_config(gpu, c3_case, variant, split):
    x, w, dy, ey, er, *_ = c3_case
    y, rstd = fwd(x, w, variant, split, gpu)
    np.testing.assert_allclose(rstd, er, **FP32)
    np.testing.assert_allclose(y, ey, **BF16)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 16), ("read", 0)])
def test_rmsnorm_bwd_full_config(gpu, c3_case, variant, split):
    x, w, dy, _, _, r32, edx, edw = c3_case
    dx, dw = bwd(x, w, dy, r32, variant, split, gpu)
    np.testing.assert_allclose(dw, edw, **FP32)
    np.testing.assert_allclose(dx, edx, **BF16)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 18), ("split", 37)])
def test_rmsnorm_bwd_back_to_back_launches(gpu, c3_case, variant, split):
    """Launches queued with no host synchronisation between them (as a
    training step issues them): every group of the split kernel must be
    resident at once, or a group whose last members wait for dispatch
    stalls until the exchange watchdog expires.  The grid is sized to one
    resident wave; this checks no launch raises the watchdog and the last
    result is still exact."""
    x, w, dy, _, _, r32, edx, edw = c3_case
    ins = [t.to(gpu) for t in (x, w, dy)] + [torch.from_numpy(r32).to(gpu)]
    dx = torch.empty_like(ins[0])
    dw = torch.empty(x.shape[1], dtype=torch.float32, device=gpu)
    cfg = hip_lib.make_cfg(variant, split)
    for _ in range(6):
        hip_lib.rmsnorm_bwd(*ins, dx, dw, cfg)
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    np.testing.assert_allclose(dw.cpu().numpy(), edw, **FP32)
    np.testing.assert_allclose(dx.float().cpu().numpy(), edx, **BF16)


def fused(x, w, dy, variant, split, gpu):
    ins = [t.to(gpu) for t in (x, w, dy)]
    y = torch.empty_like(ins[0])
    rstd = torch.full((x.shape[0],), float("nan"), device=gpu)
    dx = torch.empty_like(ins[0])
    dw = torch.full((x.shape[1],), float("nan"), device=gpu)
    hip_lib.rmsnorm_fwd_bwd(*ins, y, rstd, dx, dw, EPS, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return (y.float().cpu().numpy(), rstd.cpu().numpy(), dx.float().cpu().numpy(),
            dw.cpu().numpy())


def check_fused(x, w, dy, y, rstd, dx, dw):
    """rstd against the float64 forward; y, dx and dweight against the
    oracle given the kernel's own fp32 rstd (as the backward tests give it
    the rstd input): a 1-ulp difference of rstd in a row moves dweight's
    cancelling columns by more than fp32's atol, and is no error of the
    backward arithmetic."""
    xf, wf, dyf = x.float().numpy(), w.float().numpy(), dy.float().numpy()
    _, er = ref.rmsnorm_fwd(xf, wf, EPS)
    np.testing.assert_allclose(rstd, er, **FP32)
    edx, edw = ref.rmsnorm_bwd(xf, wf, dyf, rstd)
    np.testing.assert_allclose(dw, edw, **FP32)
    np.testing.assert_allclose(y, xf.astype(np.float64) * rstd[:, None] * wf, **BF16)
    np.testing.assert_allclose(dx, edx, **BF16)


@pytest.mark.parametrize("shape,variant,split", [((16, 8192), "auto", 0), ((5, 65536), "split", 8),
                                                 ((77, 65544), "auto", 0), ((300, 16384), "split", 2),
                                                 ((9, 4096), "read", 0), ((33, 24), "auto", 0),
                                                 ((130, 262144), "auto", 0)])
def test_rmsnorm_fwd_bwd_shapes(gpu, shape, variant, split):
    """The fused call: one member per row (8192 columns), ragged last members
    (65544 = 8193 vectors over 16), more rows than groups, the two-call READ
    path, a row too narrow for 16-byte vectors (AUTO takes the two calls),
    and 32 members at 262144 columns."""
    print(f"rmsnorm_fwd_bwd {variant} P={split} shape={shape}", flush=True)
    x, w, dy = SPEC.make_inputs(*shape, seed=shape[0] + 3)
    check_fused(x, w, dy, *fused(x, w, dy, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 32), ("read", 0)])
def test_rmsnorm_fwd_bwd_full_config(gpu, c3_case, variant, split):
    x, w, dy, *_ = c3_case
    check_fused(x, w, dy, *fused(x, w, dy, variant, split, gpu))


def test_rmsnorm_fwd_bwd_back_to_back_and_rejections(gpu, c3_case):
    x, w, dy, ey, er, r32, edx, edw = c3_case
    ins = [t.to(gpu) for t in (x, w, dy)]
    y, rstd, dx, dw = hip_lib.allocate_outputs("rmsnorm_fwd_bwd", ins)
    cfg = hip_lib.make_cfg("auto")
    for _ in range(6):
        hip_lib.rmsnorm_fwd_bwd(*ins, y, rstd, dx, dw, EPS, cfg)
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    check_fused(x, w, dy, y.float().cpu().numpy(), rstd.cpu().numpy(), dx.float().cpu().numpy(),
                dw.cpu().numpy())
    for variant, split in (("staged", 0), ("split", 8), ("split", 64)):
        with pytest.raises(hip_lib.CreditError) as err:
            hip_lib.rmsnorm_fwd_bwd(*ins, y, rstd, dx, dw, EPS, hip_lib.make_cfg(variant, split))
        assert err.value.status == -4
