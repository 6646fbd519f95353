"""GPU parity of credit_ffn_rmsnorm_gelu_bwd_bf16: dx, dW1, dW2 of
out = x + GELU_tanh(RMSNorm(x) @ W1) @ W2 for an upstream gradient dout,
against the float64 oracle (oracle.reference.ffn_rmsnorm_gelu_backward with
the GPU path's bf16 roundings of a, u, h and du).

Tolerance: bf16 outputs within rtol 1e-2 of each element plus 1e-2 of the
tensor's largest magnitude (dW entries are sums over the rows and span a wide
range; a flat atol of 1e-2 would not scale with them).  A wrong operand
layout or transpose scrambles every output by O(1) of that scale.  Shapes
cover the 128-tile GEMMs, the 256-tile GEMMs and mixtures of both; at the
full C5 shape sampled rows of dx and sampled columns of dW1 / dW2 are checked
(each depends only on its own rows / columns of the intermediates), and every
element against a float32 restatement on the GPU (torch_fp32_backward), itself
held to float64 on sampled rows and columns."""
import ctypes

import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import make_ffn_backward_inputs
from oracle import reference as ref

pytestmark = pytest.mark.gpu

EPS = 1.0e-6


def close(got, exp, name):
    """bf16 parity: rtol 1e-2 and atol 1e-2 for dx (O(1) per element, the
    flat tolerance of every bf16 output); for the weight gradients, sums over
    all rows whose magnitude spans orders, atol 1e-2 times the largest
    expected element."""
    got = np.asarray(got, np.float64)
    scale = 1.0 if name.startswith("dx") else np.abs(exp).max()
    excess = np.abs(got - exp) - (1e-2 * np.abs(exp) + 1e-2 * scale)
    assert np.all(excess <= 0), (f"{name}: max excess {excess.max():.3e} (scale {scale:.3e}) "
                                 f"at {np.unravel_index(excess.argmax(), excess.shape)}")


def make(rows, d, f, seed):
    g = torch.Generator().manual_seed(seed)
    return make_ffn_backward_inputs(rows, d, g, ffn_dim=f)


def run_bwd(x, w1, w2, dout, gpu):
    xs, ds = x.to(gpu), dout.to(gpu)
    w1l = hip_lib.linear_layout(w1.to(gpu))  # [f, d]
    w2l = hip_lib.linear_layout(w2.to(gpu))  # [d, f]
    dx = torch.full_like(xs, float("nan"))
    dw1 = torch.full_like(w1l, float("nan"))
    dw2 = torch.full_like(w2l, float("nan"))
    hip_lib.ffn_backward(xs, w1l, w2l, ds, dx, dw1, dw2, EPS, hip_lib.make_cfg())
    torch.cuda.synchronize()
    # Back to the BASELINE layouts of the oracle: dW1 [d, f], dW2 [f, d].
    return (dx.float().cpu().numpy(), dw1.float().cpu().numpy().T,
            dw2.float().cpu().numpy().T)


def oracle(x, w1, w2, dout):
    return ref.ffn_rmsnorm_gelu_backward(x.float().numpy(), w1.float().numpy(),
                                         w2.float().numpy(), dout.float().numpy(), EPS)


# (128, 128, 128) .. (384, 512, 256): 128-tile GEMMs throughout;
# (512, 512, 1024): the f-wide GEMMs on 256 tiles, da on 128 tiles;
# (1024, 512, 2048): every GEMM on 256 tiles; (128, 12288, 256) and
# (128, 20480, 128): rows wider than C5's for the dx row kernel.
@pytest.mark.parametrize("rows,d,f", [(128, 128, 128), (128, 256, 384), (256, 128, 512),
                                      (384, 512, 256), (512, 512, 1024), (1024, 512, 2048),
                                      (128, 12288, 256), (128, 20480, 128)])
def test_ffn_backward_small_shapes(gpu, rows, d, f):
    print(f"ffn_backward rows={rows} d={d} f={f}", flush=True)
    x, w1, w2, dout = make(rows, d, f, seed=rows + d + f)
    got = run_bwd(x, w1, w2, dout, gpu)
    for g, e, name in zip(got, oracle(x, w1, w2, dout), ("dx", "dW1", "dW2")):
        close(g, e, name)


def test_ffn_backward_zero_rows(gpu):
    """No rows: dx is empty and both weight gradients are exactly zero."""
    _, w1, w2, _ = make(128, 128, 256, seed=9)
    w1l = hip_lib.linear_layout(w1.to(gpu))
    w2l = hip_lib.linear_layout(w2.to(gpu))
    x = torch.empty(0, 128, dtype=torch.bfloat16, device=gpu)
    dx = torch.empty_like(x)
    dw1 = torch.full_like(w1l, 1.0)
    dw2 = torch.full_like(w2l, 1.0)
    hip_lib.ffn_backward(x, w1l, w2l, x, dx, dw1, dw2, EPS, hip_lib.make_cfg())
    torch.cuda.synchronize()
    assert not bool(dw1.any()) and not bool(dw2.any())


def test_ffn_backward_rejects_bad_shapes(gpu):
    x, w1, w2, dout = make(128, 128, 256, seed=10)
    xs, ds = x.to(gpu), dout.to(gpu)
    w1l = hip_lib.linear_layout(w1.to(gpu))
    w2l = hip_lib.linear_layout(w2.to(gpu))
    dx, dw1, dw2 = torch.empty_like(xs), torch.empty_like(w1l), torch.empty_like(w2l)
    with pytest.raises(hip_lib.CreditError):  # rows not a multiple of 128
        hip_lib.ffn_backward(xs[:100], w1l, w2l, ds[:100], dx[:100], dw1, dw2, EPS,
                             hip_lib.make_cfg())
    with pytest.raises(ValueError):  # dw1 in the wrong layout
        hip_lib.ffn_backward(xs, w1l, w2l, ds, dx, dw2, dw1, EPS, hip_lib.make_cfg())


def test_ffn_backward_full_shape_samples(gpu):
    """C5 (4096 x 8192 x 28672): 8 rows of dx and 4 columns each of dW1 and
    dW2 against the oracle restricted to what they depend on."""
    x, w1, w2, dout = make(4096, 8192, 28672, seed=0)
    dx, dw1, dw2 = run_bwd(x, w1, w2, dout, gpu)
    assert np.isfinite(dx).all() and np.isfinite(dw1).all() and np.isfinite(dw2).all()
    X = x.float().numpy().astype(np.float64)
    W1 = w1.float().numpy().astype(np.float64)
    W2 = w2.float().numpy().astype(np.float64)
    G = dout.float().numpy().astype(np.float64)
    rstd = 1.0 / np.sqrt((X * X).mean(-1, keepdims=True) + EPS)
    a = ref.round_bf16(X * rstd)
    # dx rows: each needs only its own row of u, du.
    rows = np.array([0, 1, 777, 2048, 3000, 4000, 4094, 4095])
    ex, _, _ = ref.ffn_rmsnorm_gelu_backward(X[rows], W1, W2, G[rows], EPS)
    close(dx[rows], ex, "dx rows")
    # dW2[f0, :] = h[:, f0]^T dout and dW1[:, f0] = a^T du[:, f0]: one column
    # of u (all rows) each.
    for f0 in (0, 5, 10000, 28671):
        u = a @ W1[:, f0]
        h = ref.round_bf16(ref.gelu_tanh(u))
        du = ref.round_bf16((G @ W2[f0, :]) * ref.gelu_tanh_grad(ref.round_bf16(u)))
        close(dw2[f0], h @ G, f"dW2 row {f0}")
        close(dw1[:, f0], a.T @ du, f"dW1 column {f0}")


def torch_fp32_backward(x, w1, w2, dout, gpu):
    """(dx, dW1 [d, f], dW2 [f, d]) in float32 on the GPU with the 256-tile
    path's arithmetic and roundings: u = rstd (x @ W1) from the fp32 product
    (stored as bf16 u, h = bf16(GELU(u)) taken before that rounding), du =
    bf16((dout W2^T) GELU'(bf16 u)), a = bf16(x rstd) for dW1, da = du W1^T in
    fp32, dx = dout + rstd (da - x^ mean(da x^)).  Full float32 products."""
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        X, G = x.to(gpu).float(), dout.to(gpu).float()
        W1, W2 = w1.to(gpu).float(), w2.to(gpu).float()
        rstd = torch.rsqrt((X * X).mean(dim=1, keepdim=True) + EPS)
        uf = (X @ W1) * rstd
        h = torch.nn.functional.gelu(uf, approximate="tanh").to(torch.bfloat16).float()
        u = uf.to(torch.bfloat16).float()
        del uf
        c = 0.7978845608028654
        t = torch.tanh(c * (u + 0.044715 * u ** 3))
        gp = 0.5 * (1.0 + t) + 0.5 * u * (1.0 - t * t) * c * (1.0 + 3.0 * 0.044715 * u * u)
        del t, u
        du = ((G @ W2.t()) * gp).to(torch.bfloat16).float()
        del gp
        dw2 = h.t() @ G
        del h
        ahat = X * rstd
        dw1 = ahat.to(torch.bfloat16).float().t() @ du
        da = du @ W1.t()
        dx = G + rstd * (da - ahat * (da * ahat).mean(dim=1, keepdim=True))
        return dx, dw1, dw2
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev


def close_gpu(got, exp, name):
    """close() on device tensors: |got - exp| <= 1e-2 |exp| + 1e-2 (dx) or
    + 1e-2 max|exp| (the weight gradients)."""
    scale = 1.0 if name.startswith("dx") else float(exp.abs().max())
    excess = (got - exp).abs() - (1e-2 * exp.abs() + 1e-2 * scale)
    worst = int(excess.argmax())
    assert float(excess.max()) <= 0, (
        f"{name}: max excess {float(excess.max()):.3e} (scale {scale:.3e}) at "
        f"{np.unravel_index(worst, tuple(exp.shape))}")


def test_ffn_backward_full_shape_every_element(gpu):
    """C5 (4096 x 8192 x 28672): every element of dx, dW1 and dW2 against
    torch_fp32_backward, itself checked against float64 on 2 columns each of
    dW1 and dW2 (to a tenth of the tolerance) and against the float64 oracle
    on 4 rows of dx (to a third)."""
    x, w1, w2, dout = make(4096, 8192, 28672, seed=0)
    print("ffn_backward C5 every element", flush=True)
    xs, ds = x.to(gpu), dout.to(gpu)
    w1l = hip_lib.linear_layout(w1.to(gpu))
    w2l = hip_lib.linear_layout(w2.to(gpu))
    dx = torch.full_like(xs, float("nan"))
    dw1 = torch.full_like(w1l, float("nan"))
    dw2 = torch.full_like(w2l, float("nan"))
    hip_lib.ffn_backward(xs, w1l, w2l, ds, dx, dw1, dw2, EPS, hip_lib.make_cfg())
    torch.cuda.synchronize()
    del w1l, w2l
    ex, ew1, ew2 = torch_fp32_backward(x, w1, w2, dout, gpu)
    # The float32 reference against the float64 oracle where that is cheap.
    X = x.float().numpy().astype(np.float64)
    W1 = w1.float().numpy().astype(np.float64)
    W2 = w2.float().numpy().astype(np.float64)
    Gd = dout.float().numpy().astype(np.float64)
    rows = np.array([0, 2047, 2048, 4095])
    ox, _, _ = ref.ffn_rmsnorm_gelu_backward(X[rows], W1, W2, Gd[rows], EPS)
    rstd = 1.0 / np.sqrt((X * X).mean(-1, keepdims=True) + EPS)
    a = ref.round_bf16(X * rstd)
    for f0 in (7, 20000):
        u = (X @ W1[:, f0]) * rstd[:, 0]
        h = ref.round_bf16(ref.gelu_tanh(u))
        du = ref.round_bf16((Gd @ W2[f0, :]) * ref.gelu_tanh_grad(ref.round_bf16(u)))
        e2, e1 = ew2[f0].cpu().numpy(), ew1[:, f0].cpu().numpy()
        o2, o1 = h @ Gd, a.T @ du
        np.testing.assert_array_less(np.abs(e2 - o2), 1e-3 * np.abs(o2) + 1e-3 * np.abs(o2).max())
        np.testing.assert_array_less(np.abs(e1 - o1), 1e-3 * np.abs(o1) + 1e-3 * np.abs(o1).max())
    # The oracle's dx rounds a = x rstd to bf16 before the u GEMM (the 128-tile
    # arithmetic); the reference, like the 256-tile path, scales the fp32
    # product: the two differ by up to ~1.3e-3 of the scale through du's
    # rounding, so this pin is 3e-3, a third of the test's tolerance.
    exr = ex[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    np.testing.assert_array_less(np.abs(exr - ox), 3e-3 * np.abs(ox) + 3e-3 * np.abs(ox).max())
    close_gpu(dx.float(), ex, "dx")
    close_gpu(dw1.float().t(), ew1, "dW1")
    close_gpu(dw2.float().t(), ew2, "dW2")


# ------------------------------------------------ saved-activation form --


def run_train_forward(x, w1l, w2l, gpu):
    """The training forward on device tensors (w1l [f, d], w2l [d, f])."""
    rows, f = x.shape[0], w1l.shape[0]
    out = torch.full_like(x, float("nan"))
    rstd = torch.full((rows,), float("nan"), device=gpu)
    u = torch.full((rows, f), float("nan"), device=gpu, dtype=torch.bfloat16)
    h = torch.full_like(u, float("nan"))
    hip_lib.ffn_train_forward(x, w1l, w2l, out, rstd, u, h, EPS, hip_lib.make_cfg())
    return out, rstd, u, h


@pytest.mark.parametrize("rows,d,f", [(128, 128, 256), (256, 128, 512), (512, 512, 1024),
                                      (1024, 512, 2048)])
def test_ffn_train_forward(gpu, rows, d, f):
    """out bit-identical to the plain forward; rstd, u and h against the
    float64 oracle (u and h with the arithmetic of the GEMM path the shape
    takes: bf16(x rstd) on 128 tiles, rstd on the fp32 sum on 256 tiles)."""
    print(f"ffn train forward rows={rows} d={d} f={f}", flush=True)
    x, w1, w2, _ = make(rows, d, f, seed=3 * rows + f)
    xs = x.to(gpu)
    w1l, w2l = hip_lib.linear_layout(w1.to(gpu)), hip_lib.linear_layout(w2.to(gpu))
    out, rstd, u, h = run_train_forward(xs, w1l, w2l, gpu)
    plain = torch.empty_like(xs)
    hip_lib.ffn(xs, w1l, w2l, plain, EPS, hip_lib.make_cfg())
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    X = x.float().numpy().astype(np.float64)
    ers = 1.0 / np.sqrt((X * X).mean(-1) + EPS)
    np.testing.assert_allclose(rstd.cpu().numpy(), ers, rtol=1e-5, atol=1e-6)
    big = d % 256 == 0 and f % 256 == 0
    a = X * ers[:, None] if big else ref.round_bf16(X * ers[:, None])
    eu = a @ w1.float().numpy().astype(np.float64)
    close(u.float().cpu().numpy(), eu, "u")
    close(h.float().cpu().numpy(), ref.gelu_tanh(eu), "h")


@pytest.mark.parametrize("rows,d,f", [(128, 128, 128), (256, 128, 512), (384, 512, 256),
                                      (512, 512, 1024), (1024, 512, 2048), (4096, 8192, 28672)])
def test_ffn_backward_saved_is_bit_identical(gpu, rows, d, f):
    """The backward from the training forward's rstd, u and h gives the
    recomputing backward's bits: the saved u and h are the recomputed ones,
    and h read as a [K, N] operand feeds the dW2 GEMM the same values in the
    same order as h^T.  Includes the full C5 shape."""
    print(f"ffn_backward_saved rows={rows} d={d} f={f}", flush=True)
    x, w1, w2, dout = make(rows, d, f, seed=rows + 2 * d + f)
    xs, ds = x.to(gpu), dout.to(gpu)
    w1l, w2l = hip_lib.linear_layout(w1.to(gpu)), hip_lib.linear_layout(w2.to(gpu))
    _, rstd, u, h = run_train_forward(xs, w1l, w2l, gpu)
    outs = []
    for saved in (False, True):
        dx = torch.full_like(xs, float("nan"))
        dw1 = torch.full_like(w1l, float("nan"))
        dw2 = torch.full_like(w2l, float("nan"))
        if saved:
            hip_lib.ffn_backward_saved(xs, w1l, w2l, ds, rstd, u, h, dx, dw1, dw2,
                                       hip_lib.make_cfg())
        else:
            hip_lib.ffn_backward(xs, w1l, w2l, ds, dx, dw1, dw2, EPS, hip_lib.make_cfg())
        torch.cuda.synchronize()
        outs.append((dx, dw1, dw2))
    for name, a, b in zip(("dx", "dw1", "dw2"), *outs):
        assert not torch.isnan(b.float()).any(), name
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
    del outs, u, h
    torch.cuda.empty_cache()


def test_ffn_backward_saved_rejects_bad_shapes(gpu):
    x, w1, w2, dout = make(128, 128, 256, seed=11)
    xs, ds = x.to(gpu), dout.to(gpu)
    w1l, w2l = hip_lib.linear_layout(w1.to(gpu)), hip_lib.linear_layout(w2.to(gpu))
    _, rstd, u, h = run_train_forward(xs, w1l, w2l, gpu)
    dx, dw1, dw2 = torch.empty_like(xs), torch.empty_like(w1l), torch.empty_like(w2l)
    with pytest.raises(ValueError):  # u of the wrong width
        hip_lib.ffn_backward_saved(xs, w1l, w2l, ds, rstd, u[:, :128], h, dx, dw1, dw2,
                                   hip_lib.make_cfg())
    with pytest.raises(hip_lib.CreditError):  # misaligned h (checked in the library)
        hv = h.view(-1)[1:].view(-1)[: h.numel() - 8]
        lib = hip_lib.load_library()
        st = lib.credit_ffn_rmsnorm_gelu_bwd_saved_bf16(
            xs.data_ptr(), w1l.data_ptr(), w2l.data_ptr(), ds.data_ptr(), rstd.data_ptr(),
            u.data_ptr(), hv.data_ptr(), dx.data_ptr(), dw1.data_ptr(), dw2.data_ptr(), 128, 128,
            256, ctypes.byref(hip_lib.make_cfg()))
        hip_lib.check(st, "credit_ffn_rmsnorm_gelu_bwd_saved_bf16")


# ------------------------------------------------ [in, out] weight layout --


@pytest.mark.parametrize("rows,d,f", [(128, 128, 256), (256, 128, 512), (384, 512, 256),
                                      (512, 512, 1024), (1024, 512, 2048), (4096, 8192, 28672)])
def test_ffn_backward_in_out_layout_is_bit_identical(gpu, rows, d, f):
    """The [in, out] entry points (w1 [d, f], w2 [f, d] read as they are,
    gradients returned in that layout) against the nn.Linear ones on the
    transposed weights: the training forward's out, rstd, u and h, and dx,
    dW1^T and dW2^T of both backward forms, bit for bit.  The weight-gradient
    GEMMs take their operands the other way round there (a^T du, h^T dout;
    the saved form's dW2 stored transposed), which changes neither the
    products nor their order.  Includes the full C5 shape."""
    print(f"ffn_backward [in, out] rows={rows} d={d} f={f}", flush=True)
    x, w1, w2, dout = make(rows, d, f, seed=5 * rows + d + f)
    xs, ds = x.to(gpu), dout.to(gpu)
    w1k, w2k = w1.to(gpu).contiguous(), w2.to(gpu).contiguous()   # [d, f], [f, d]
    w1l, w2l = hip_lib.linear_layout(w1k), hip_lib.linear_layout(w2k)  # [f, d], [d, f]
    cfg = hip_lib.make_cfg()

    def train(wa, wb, kn):
        out = torch.full_like(xs, float("nan"))
        rstd = torch.full((rows,), float("nan"), device=gpu)
        u = torch.full((rows, f), float("nan"), device=gpu, dtype=torch.bfloat16)
        h = torch.full_like(u, float("nan"))
        hip_lib.ffn_train_forward(xs, wa, wb, out, rstd, u, h, EPS, cfg, kn=kn)
        return out, rstd, u, h

    def backward(wa, wb, kn, saved):
        dx = torch.full_like(xs, float("nan"))
        dw1, dw2 = torch.full_like(wa, float("nan")), torch.full_like(wb, float("nan"))
        if saved is None:
            hip_lib.ffn_backward(xs, wa, wb, ds, dx, dw1, dw2, EPS, cfg, kn=kn)
        else:
            hip_lib.ffn_backward_saved(xs, wa, wb, ds, *saved[1:], dx, dw1, dw2, cfg, kn=kn)
        return dx, dw1, dw2

    def same(a, b, name):
        assert not torch.isnan(a.float()).any(), name
        assert torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16)), (
            f"{name}: max |diff| {float((a.float() - b.float()).abs().max()):.3e}")

    lin, kn = train(w1l, w2l, False), train(w1k, w2k, True)
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "rstd", "u", "h"), kn, lin):
        same(a, b, f"train forward {name}")
    for saved in (None, "saved"):
        ref_g = backward(w1l, w2l, False, None if saved is None else lin)
        got_g = backward(w1k, w2k, True, None if saved is None else kn)
        torch.cuda.synchronize()
        same(got_g[0], ref_g[0], f"{saved} dx")
        same(got_g[1], ref_g[1].t(), f"{saved} dW1")
        same(got_g[2], ref_g[2].t(), f"{saved} dW2")
        del ref_g, got_g
    del lin, kn
    torch.cuda.empty_cache()
