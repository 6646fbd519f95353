"""GPU parity of the reference's remaining wide-row workloads against the
float64 oracle: credit_lars_momentum_f32 (dsmem_eval/workloads.py:136-143),
credit_weighted_var_bwd_f32 (:72-85) and credit_pearson_bwd_f32 (:96-112).

Tolerance: fp32 outputs within rtol 1e-5 / atol 1e-6 of the float64 oracle
(the reference itself asks 3e-3 or 3e-2, dsmem_eval/workloads.py:164-201).
LARS's update u = 0.9 m + g + 0.01 w is also checked bit-exact against the
same expression in float32 (the reference's torch function rounds each
operation in fp32)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

FP32 = dict(rtol=1e-5, atol=1e-6)
VARIANTS = [("auto", 0), ("staged", 0), ("read", 0), ("split", 2), ("split", 3), ("split", 8)]
SHAPES = [(16, 4096), (5, 12), (3, 65536), (9, 4100), (33, 1024), (2, 4)]
UNALIGNED = [(7, 4097), (3, 1), (4, 30)]


def _gpu(ts, gpu):
    return [torch.as_tensor(t).to(gpu) for t in ts]


PARTIALS = {"lars_momentum": 2, "weighted_var_backward": 5, "pearson_backward": 5}
# f32x4 one member holds under an explicit SPLIT where it exceeds the STAGED
# width (the weighted-variance 512-lane 16-vector slice shape).
SPLIT_CAP = {"weighted_var_backward": 8192}


def supported(name, variant, split, cols):
    """Whether the library takes this variant at this width: STAGED up to
    the workload's staged width, SPLIT while every member's slice fits one
    workgroup and members x partials fit one exchange."""
    cap = WORKLOADS[name].staged_max_cols // 4
    nvec = cols // 4
    if variant in ("auto", "read"):
        return True
    if cols % 4:
        return False
    if variant == "staged":
        return nvec <= cap
    p = min(split, nvec)
    chunk = -(-nvec // p)
    members = -(-nvec // chunk)
    return chunk <= SPLIT_CAP.get(name, cap) and members * PARTIALS[name] <= 64


def run_or_reject(name, variant, split, cols, fn):
    """fn() when the variant is supported, else the library must refuse it."""
    if supported(name, variant, split, cols):
        return fn()
    with pytest.raises(hip_lib.CreditError):
        fn()
    return None


# ------------------------------------------------------------------- LARS --


def lars(w, g, m, variant, split, gpu):
    ws, gs, ms = _gpu((w, g, m), gpu)
    wo = torch.full_like(ws, float("nan"))
    uo = torch.full_like(ws, float("nan"))
    hip_lib.lars_momentum(ws, gs, ms, wo, uo, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return wo.cpu().numpy(), uo.cpu().numpy()


def check_lars(w, g, m, wo, uo):
    w, g, m = (np.asarray(t, dtype=np.float32) for t in (w, g, m))
    u32 = (np.float32(0.9) * m + g) + np.float32(0.01) * w
    assert np.array_equal(uo, u32), "update is not bit-exact with the fp32 expression"
    ew, eu = ref.lars_momentum(w, g, m)
    np.testing.assert_allclose(uo, eu, **FP32)
    np.testing.assert_allclose(wo, ew, **FP32)


@pytest.mark.parametrize("variant,split", VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_lars_shapes(gpu, variant, split, shape):
    print(f"lars {variant} P={split} shape={shape}", flush=True)
    w, g, m = WORKLOADS["lars_momentum"].make_inputs(*shape, seed=71)
    got = run_or_reject("lars_momentum", variant, split, shape[1],
                        lambda: lars(w, g, m, variant, split, gpu))
    if got is not None:
        check_lars(w, g, m, *got)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0)])
@pytest.mark.parametrize("shape", UNALIGNED)
def test_lars_unaligned_widths(gpu, variant, split, shape):
    w, g, m = WORKLOADS["lars_momentum"].make_inputs(*shape, seed=72)
    check_lars(w, g, m, *lars(w, g, m, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 8), ("split", 16), ("read", 0)])
def test_lars_wide_rows(gpu, variant, split):
    w, g, m = WORKLOADS["lars_momentum"].make_inputs(4, 262144, seed=73)
    check_lars(w, g, m, *lars(w, g, m, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("staged", 0), ("split", 2), ("read", 0)])
def test_lars_zero_rows_and_hash_inputs(gpu, variant, split):
    """The CUDA workload's own inputs (lars_momentum.cu:257-275), with an
    all-zero row (w = u = 0: trust 0, w' = 0) and a row with zero update."""
    w, g, m = ref.lars_momentum_init(16, 8192)
    w[3] = g[3] = m[3] = 0.0
    m[5] = 0.0
    g[5] = -np.float32(0.01) * w[5]  # 0.01 w + g rounds to 0 or a few ulp
    check_lars(w, g, m, *lars(w, g, m, variant, split, gpu))


# ------------------------------------------------- weighted variance bwd --


def wvar(x, w, dy, variant, split, gpu, eps=1e-5):
    xs, ws, ds = _gpu((x, w, dy), gpu)
    dx = torch.full_like(xs, float("nan"))
    hip_lib.weighted_var_backward(xs, ws, ds, dx, eps, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return dx.cpu().numpy()


WVAR_VARIANTS = [("auto", 0), ("staged", 0), ("read", 0), ("split", 2), ("split", 3),
                 ("split", 12)]


@pytest.mark.parametrize("variant,split", WVAR_VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_weighted_var_shapes(gpu, variant, split, shape):
    print(f"weighted_var {variant} P={split} shape={shape}", flush=True)
    x, w, dy = WORKLOADS["weighted_var_backward"].make_inputs(*shape, seed=81)
    got = run_or_reject("weighted_var_backward", variant, split, shape[1],
                        lambda: wvar(x, w, dy, variant, split, gpu))
    if got is not None:
        np.testing.assert_allclose(got, ref.weighted_var_backward(x, w, dy), **FP32)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0)])
@pytest.mark.parametrize("shape", [(7, 4097), (3, 5), (4, 30)])
def test_weighted_var_unaligned_widths(gpu, variant, split, shape):
    x, w, dy = WORKLOADS["weighted_var_backward"].make_inputs(*shape, seed=82)
    np.testing.assert_allclose(wvar(x, w, dy, variant, split, gpu),
                               ref.weighted_var_backward(x, w, dy), **FP32)


def test_weighted_var_single_column(gpu):
    """cols = 1: dx = inv_std dy eps / (w + eps), about 1e-5 of the two fp32
    terms it is the difference of (inv_std ~ 316), so fp32 evaluation of the
    reference formula keeps only ~2 digits; checked at the reference's own
    tolerance, 3e-2 (dsmem_eval/workloads.py:172-173)."""
    x, w, dy = WORKLOADS["weighted_var_backward"].make_inputs(3, 1, seed=84)
    np.testing.assert_allclose(wvar(x, w, dy, "auto", 0, gpu),
                               ref.weighted_var_backward(x, w, dy), rtol=3e-2, atol=3e-2)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 8), ("split", 12), ("read", 0)])
def test_weighted_var_wide_and_shifted_rows(gpu, variant, split):
    """Wide rows, one of them shifted by 1000 (the one-pass sums are taken
    about the row's first element: no cancellation from the offset)."""
    x, w, dy = WORKLOADS["weighted_var_backward"].make_inputs(4, 131072, seed=83)
    x[1] += 1000.0
    x[2] *= 1e-3
    np.testing.assert_allclose(wvar(x, w, dy, variant, split, gpu),
                               ref.weighted_var_backward(x, w, dy), **FP32)


@pytest.mark.parametrize("variant,split", [("split", 8), ("split", 12), ("split", 6),
                                           ("auto", 0)])
def test_weighted_var_262144_columns(gpu, variant, split):
    """The widest swept width: an explicit SPLIT of 8 or 12 members takes the
    512-lane 16-vector slice shape (32768 and 21848 columns per member), 6
    members are too few (43692 > 32768 columns each) and are refused, AUTO stays
    on the 4096-vector shapes (16 members x 5 partials exceed one exchange:
    the READ kernel).  Row 1 is shifted by 1000."""
    print(f"weighted_var 262144 {variant} P={split}", flush=True)
    x, w, dy = WORKLOADS["weighted_var_backward"].make_inputs(3, 262144, seed=85)
    x[1] += 1000.0
    got = run_or_reject("weighted_var_backward", variant, split, 262144,
                        lambda: wvar(x, w, dy, variant, split, gpu))
    assert (got is None) == (split == 6)
    if got is not None:
        np.testing.assert_allclose(got, ref.weighted_var_backward(x, w, dy), **FP32)


def test_weighted_var_hash_inputs_and_rejects(gpu):
    x, w, dy = ref.weighted_var_backward_init(16, 16384)
    np.testing.assert_allclose(wvar(x, w, dy, "auto", 0, gpu),
                               ref.weighted_var_backward(x, w, dy), **FP32)
    xs, ws, ds = _gpu((x, w, dy), gpu)
    dx = torch.empty_like(xs)
    with pytest.raises(hip_lib.CreditError):  # 13 members x 5 partials > 64
        hip_lib.weighted_var_backward(xs, ws, ds, dx, 1e-5, hip_lib.make_cfg("split", 13))
    with pytest.raises(hip_lib.CreditError):
        hip_lib.weighted_var_backward(xs, ws, ds, dx, 0.0, hip_lib.make_cfg())


# ------------------------------------------------------- pearson backward --


def pearson(x, y, grad, variant, split, gpu, eps=1e-6):
    xs, ys, gs = _gpu((x, y, grad), gpu)
    dx = torch.full_like(xs, float("nan"))
    dy = torch.full_like(xs, float("nan"))
    hip_lib.pearson_backward(xs, ys, gs, dx, dy, eps, hip_lib.make_cfg(variant, split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    return dx.cpu().numpy(), dy.cpu().numpy()


def check_pearson(x, y, grad, got):
    """rtol 1e-5, with atol 1e-6 taken relative to the row's largest term
    grad * yc / sqrt(vx vy): the gradients scale as 1/N (|dx| ~ 1e-5 at
    N = 65536), where a flat atol of 1e-6 would accept 10% errors, and they
    vanish as the difference of two such terms on a perfectly correlated
    row."""
    ex, ey = ref.pearson_backward(x, y, grad)
    x64, y64 = np.asarray(x, np.float64), np.asarray(y, np.float64)
    xc = x64 - x64.mean(-1, keepdims=True)
    yc = y64 - y64.mean(-1, keepdims=True)
    inv = 1.0 / np.sqrt(((xc * xc).sum(-1, keepdims=True) + 1e-6) * ((yc * yc).sum(-1, keepdims=True) + 1e-6))
    g64 = np.abs(np.asarray(grad, np.float64))
    for g, e, c in zip(got, (ex, ey), (yc, xc)):
        scale = (g64 * np.abs(c) * inv).max(axis=-1, keepdims=True)
        err = np.abs(g - e) - (1e-5 * np.abs(e) + 1e-6 * scale)
        assert np.all(err <= 0), f"max excess {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("variant,split", WVAR_VARIANTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_pearson_shapes(gpu, variant, split, shape):
    print(f"pearson {variant} P={split} shape={shape}", flush=True)
    x, y, grad = WORKLOADS["pearson_backward"].make_inputs(*shape, seed=91)
    got = run_or_reject("pearson_backward", variant, split, shape[1],
                        lambda: pearson(x, y, grad, variant, split, gpu))
    if got is not None:
        check_pearson(x, y, grad, got)


@pytest.mark.parametrize("variant,split", [("auto", 0), ("read", 0)])
@pytest.mark.parametrize("shape", UNALIGNED)
def test_pearson_unaligned_widths(gpu, variant, split, shape):
    x, y, grad = WORKLOADS["pearson_backward"].make_inputs(*shape, seed=92)
    check_pearson(x, y, grad, pearson(x, y, grad, variant, split, gpu))


@pytest.mark.parametrize("variant,split", [("auto", 0), ("split", 8), ("split", 12), ("read", 0)])
def test_pearson_wide_and_shifted_rows(gpu, variant, split):
    x, y, grad = WORKLOADS["pearson_backward"].make_inputs(4, 262144, seed=93)
    x[1] += 500.0
    y[2] -= 300.0
    check_pearson(x, y, grad, pearson(x, y, grad, variant, split, gpu))


def test_pearson_hash_inputs_and_correlated_rows(gpu):
    """The CUDA workload's inputs (pearson_backward.cu:289-309) with one row
    where y = 2x + 1 (correlation 1: dx and dy vanish up to rounding)."""
    x, y, grad = ref.pearson_backward_init(17, 8192)
    y[4] = 2.0 * x[4] + 1.0
    check_pearson(x, y, grad, pearson(x, y, grad, "auto", 0, gpu))


# ------------------------------------------------------------ all three --


@pytest.mark.parametrize("name", ["lars_momentum", "weighted_var_backward", "pearson_backward"])
def test_zero_rows(gpu, name):
    ins = tuple(t.to(gpu) for t in WORKLOADS[name].make_inputs(1, 64))
    ins = tuple(t[:0] for t in ins)
    outs = hip_lib.allocate_outputs(name, ins)
    hip_lib.HIP_LAUNCHERS[name](ins, outs)
    torch.cuda.synchronize()


@pytest.mark.parametrize("name,split", [("lars_momentum", 2), ("weighted_var_backward", 4),
                                        ("pearson_backward", 8)])
def test_back_to_back(gpu, name, split):
    """Six split launches queued with no host synchronisation, each group
    taking several rows; the last result is checked."""
    cpu = WORKLOADS[name].make_inputs(2048, 16384, seed=95)
    ins = tuple(t.to(gpu) for t in cpu)
    outs = hip_lib.allocate_outputs(name, ins)
    print(f"{name} back to back P={split}", flush=True)
    for _ in range(6):
        hip_lib.HIP_LAUNCHERS[name](ins, outs, hip_lib.LaunchConfig("split", split))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    expect = {"lars_momentum": lambda: ref.lars_momentum(*(t.numpy() for t in cpu)),
              "weighted_var_backward": lambda: (ref.weighted_var_backward(*(t.numpy() for t in cpu)),),
              "pearson_backward": lambda: ref.pearson_backward(*(t.numpy() for t in cpu))}[name]()
    if name == "pearson_backward":
        check_pearson(*(t.numpy() for t in cpu), [o.cpu().numpy() for o in outs])
        return
    for got, exp in zip(outs, expect):
        np.testing.assert_allclose(got.cpu().numpy(), exp, **FP32)


@pytest.mark.parametrize("name", ["lars_momentum", "weighted_var_backward", "pearson_backward"])
def test_full_shape(gpu, name):
    """The bench shape (4096 x 65536), AUTO, a slice of rows against the
    oracle and every output finite."""
    cpu = WORKLOADS[name].make_inputs()
    ins = tuple(t.to(gpu) for t in cpu)
    outs = hip_lib.allocate_outputs(name, ins)
    hip_lib.HIP_LAUNCHERS[name](ins, outs)
    torch.cuda.synchronize()
    hip_lib.check_watchdog()
    for o in outs:
        assert bool(torch.isfinite(o).all())
    sl = tuple(t[:32].numpy() for t in cpu)
    expect = {"lars_momentum": lambda: ref.lars_momentum(*sl),
              "weighted_var_backward": lambda: (ref.weighted_var_backward(*sl),),
              "pearson_backward": lambda: ref.pearson_backward(*sl)}[name]()
    if name == "pearson_backward":
        check_pearson(*sl, [o[:32].cpu().numpy() for o in outs])
    else:
        for got, exp in zip(outs, expect):
            np.testing.assert_allclose(got[:32].cpu().numpy(), exp, **FP32)
    del ins, outs
    torch.cuda.empty_cache()
