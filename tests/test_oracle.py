"""Pins the CPU oracle (oracle/reference.py) against torch library routines
in float64, autograd, closed forms and brute force -- never against a
retyped copy of its own formula."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as ref

RNG = np.random.default_rng(7)


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


# ---------------------------------------------------------------- C1 ------


def test_row_sum_max_matches_torch():
    x = RNG.uniform(-1, 1, (8, 1000)).astype(np.float32)
    s, m = ref.row_sum_max(x)
    np.testing.assert_allclose(s, torch.sum(t64(x), -1).numpy(), rtol=1e-15, atol=1e-12)
    assert np.array_equal(m, torch.amax(torch.from_numpy(x), -1).double().numpy())


def test_row_sum_is_exact_on_tiny_rows():
    x = np.array([[1e8, 1.0, -1e8, 3.0], [0.1, 0.2, 0.3, -0.6]], dtype=np.float32)
    s, _ = ref.row_sum_max(x)
    for r in range(2):
        assert s[r] == pytest.approx(math.fsum(float(v) for v in x[r]), abs=1e-12)


def test_row_max_nan_and_inf():
    x = np.array([[1.0, np.nan, 3.0], [-np.inf, -5.0, -7.0], [np.inf, 1.0, 2.0]], dtype=np.float32)
    s, m = ref.row_sum_max(x)
    tm = torch.amax(torch.from_numpy(x), -1).numpy()
    assert np.isnan(m[0]) and np.isnan(tm[0])
    assert m[1] == tm[1] == -5.0 and m[2] == tm[2] == np.inf
    assert np.isnan(s[0])


# ---------------------------------------------------------------- C2 ------


def test_layernorm_fwd_matches_f_layer_norm():
    x = RNG.standard_normal((6, 777))
    g = RNG.normal(1, 0.02, 777)
    b = RNG.normal(0, 0.02, 777)
    y, mean, rstd = ref.layernorm_fwd(x, g, b, 1e-5)
    ty = F.layer_norm(t64(x), (777,), t64(g), t64(b), 1e-5)
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-12, atol=1e-12)
    var, tmean = torch.var_mean(t64(x), -1, unbiased=False)
    np.testing.assert_allclose(mean, tmean.numpy(), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(rstd, torch.rsqrt(var + 1e-5).numpy(), rtol=1e-13)


def test_layernorm_fwd_constant_row():
    x = np.full((1, 64), 3.25)
    g = RNG.normal(1, 0.1, 64)
    b = RNG.normal(0, 0.1, 64)
    y, mean, rstd = ref.layernorm_fwd(x, g, b, 1e-5)
    assert mean[0] == 3.25
    assert rstd[0] == pytest.approx(1 / math.sqrt(1e-5))
    np.testing.assert_allclose(y[0], b, atol=1e-15)


def test_layernorm_backward_matches_autograd():
    x = RNG.uniform(-1, 1, (5, 300))
    dy = RNG.uniform(-1, 1, (5, 300))
    g = RNG.uniform(0.75, 1.25, 300)
    tx = t64(x).requires_grad_()
    F.layer_norm(tx, (300,), t64(g), None, 1e-5).backward(t64(dy))
    np.testing.assert_allclose(ref.layernorm_backward(x, dy, g), tx.grad.numpy(), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- C3 ------


def test_rmsnorm_fwd_matches_f_rms_norm():
    x = RNG.standard_normal((4, 513))
    w = RNG.normal(1, 0.02, 513)
    y, rstd = ref.rmsnorm_fwd(x, w, 1e-6)
    np.testing.assert_allclose(y, F.rms_norm(t64(x), (513,), t64(w), 1e-6).numpy(), rtol=1e-12)
    np.testing.assert_allclose(rstd, torch.rsqrt((t64(x) ** 2).mean(-1) + 1e-6).numpy(), rtol=1e-13)


def test_rmsnorm_bwd_matches_autograd():
    x = RNG.standard_normal((7, 129))
    w = RNG.normal(1, 0.02, 129)
    dy = RNG.standard_normal((7, 129))
    tx = t64(x).requires_grad_()
    tw = t64(w).requires_grad_()
    F.rms_norm(tx, (129,), tw, 1e-6).backward(t64(dy))
    _, rstd = ref.rmsnorm_fwd(x, w, 1e-6)
    dx, dw = ref.rmsnorm_bwd(x, w, dy, rstd)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_rmsnorm_fwd_bwd_matches_autograd():
    """The fused oracle (float64 rstd) against one autograd pass of
    F.rms_norm with upstream grad dy; with the fp32 rstd it moves by about
    the fp32 rounding of rstd (relative 6e-8, more on dx entries that
    cancel: atol scaled to the largest entry)."""
    x = RNG.standard_normal((5, 257))
    w = RNG.normal(1, 0.02, 257)
    dy = RNG.standard_normal((5, 257))
    tx = t64(x).requires_grad_()
    tw = t64(w).requires_grad_()
    ty = F.rms_norm(tx, (257,), tw, 1e-6)
    ty.backward(t64(dy))
    y, rstd, dx, dw = ref.rmsnorm_fwd_bwd(x, w, dy, 1e-6, rstd_fp32=False)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)
    y32, rstd32, dx32, dw32 = ref.rmsnorm_fwd_bwd(x, w, dy, 1e-6)
    np.testing.assert_array_equal(rstd32, rstd)
    for a, b in ((y32, y), (dx32, dx), (dw32, dw)):
        np.testing.assert_allclose(a, b, rtol=2e-7, atol=2e-7 * np.abs(b).max())
        assert not np.array_equal(a, b)


# ---------------------------------------------------------------- C4 ------


def test_softmax_fwd_matches_torch():
    x = RNG.normal(0, 4, (5, 1000))
    x[RNG.random(x.shape) < 0.01] = 20.0
    p, m, lse = ref.softmax_fwd(x)
    np.testing.assert_allclose(p, torch.softmax(t64(x), -1).numpy(), rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(lse, torch.logsumexp(t64(x), -1).numpy(), rtol=1e-14)
    assert np.array_equal(m, torch.amax(t64(x), -1).numpy())


def test_softmax_fwd_spike_row():
    x = np.zeros((1, 8))
    x[0, 3] = 1000.0
    p, m, lse = ref.softmax_fwd(x)
    assert p[0, 3] == 1.0 and p[0].sum() == 1.0
    assert m[0] == 1000.0 and lse[0] == pytest.approx(1000.0)


def test_softmax_bwd_matches_autograd():
    x = RNG.normal(0, 2, (4, 200))
    dy = RNG.standard_normal((4, 200))
    tx = t64(x).requires_grad_()
    torch.softmax(tx, -1).backward(t64(dy))
    p, _, _ = ref.softmax_fwd(x)
    np.testing.assert_allclose(ref.softmax_bwd(p, dy), tx.grad.numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(ref.softmax_logits_backward(x, dy), tx.grad.numpy(), rtol=1e-10, atol=1e-14)


# ------------------------------------------------- reference workloads ----


def test_lars_special_cases():
    w = RNG.uniform(-1, 1, (3, 50))
    z = np.zeros_like(w)
    # momentum = grad = 0: update = 0.01 w, trust = 0.02|w|/(0.01|w| + 1e-6)
    new_w, upd = ref.lars_momentum(w, z, z)
    np.testing.assert_allclose(upd, 0.01 * w, rtol=1e-15)
    n = np.linalg.norm(w, axis=-1, keepdims=True)
    trust = 0.02 * n / (0.01 * n + 1e-6)
    np.testing.assert_allclose(new_w, w - 1e-3 * trust * 0.01 * w, rtol=1e-14)
    # zero weight: trust = 0, weight unchanged, update = 0.9 m + g
    m = RNG.uniform(-1, 1, w.shape)
    g = RNG.uniform(-1, 1, w.shape)
    new_w, upd = ref.lars_momentum(z, g, m)
    assert np.array_equal(new_w, z)
    np.testing.assert_allclose(upd, 0.9 * m + g, rtol=1e-15)


def test_rowwise_quant_brute_force():
    x = np.array([[0.5, -1.0, 0.25, 0.0], [0.0, 0.0, 0.0, 0.0], [3.0, 1.5, -0.75, 1.0 / 254.0]],
                 dtype=np.float32)
    q, scale = ref.rowwise_quant(x)
    assert q.dtype == np.int8
    assert q[0].tolist() == [64, -127, 32, 0]  # 63.5 rounds to even 64
    assert q[1].tolist() == [0, 0, 0, 0] and scale[1] == 0.0
    assert q[2, 0] == 127 and scale[2] == np.float32(3.0) / np.float32(127.0)
    # dequantisation error is at most half a step
    assert np.all(np.abs(q[2] * scale[2] - x[2]) <= scale[2] / 2 + 1e-7)


def test_rowwise_quant_matches_torch_operator_semantics():
    """The reference's torch function (amax, scalar / tensor, round, clamp,
    int8) on many random rows: q and scale bit-exact.  torch evaluates the
    scalar / tensor as reciprocal * scalar, which a one-step division would
    get wrong in about a quarter of the rows."""
    g = torch.Generator().manual_seed(11)
    x = (torch.rand(4096, 64, generator=g) * 2 - 1) * torch.rand(4096, 1, generator=g) * 8
    x[7] = 0.0
    # Rows whose elements land next to half-integers, (j + 0.5) * m / 127:
    # there the last bit of the reciprocal decides the rounding (a one-step
    # division gives a different q for ~12% of these elements).
    m = torch.rand(2048, 1, generator=g) * 3.5 + 0.5
    ties = (torch.arange(63, dtype=torch.float32)[None, :] + 0.5) * m / 127.0
    x = torch.cat([x, torch.cat([ties, m], dim=1)])
    max_abs = torch.amax(torch.abs(x), dim=-1, keepdim=True)
    inv = torch.where(max_abs > 0.0, 127.0 / max_abs, torch.zeros_like(max_abs))
    tq = torch.clamp(torch.round(x * inv), -127.0, 127.0).to(torch.int8)
    tscale = (max_abs / 127.0).squeeze(-1)
    q, scale = ref.rowwise_quant(x.numpy())
    assert np.array_equal(q, tq.numpy())
    assert np.array_equal(scale, tscale.numpy())


def test_weighted_var_backward_matches_autograd():
    x = RNG.uniform(-2, 2, (4, 100))
    w = RNG.uniform(0.5, 1.5, (4, 100))
    dy = RNG.uniform(-1, 1, (4, 100))
    tx = t64(x).requires_grad_()
    tw = t64(w)
    eps = 1e-5
    inv = 1.0 / (tw.sum(-1, keepdim=True) + eps)
    mean = (tw * tx).sum(-1, keepdim=True) * inv
    var = (tw * (tx - mean) ** 2).sum(-1, keepdim=True) * inv
    ((tx - mean) * torch.rsqrt(var + eps)).backward(t64(dy))
    # The reference formula drops an O(eps * mean / sum(w)^2) term.
    np.testing.assert_allclose(ref.weighted_var_backward(x, w, dy), tx.grad.numpy(), rtol=1e-6, atol=1e-8)


def test_pearson_backward_matches_autograd():
    x = RNG.uniform(-1, 1, (3, 80))
    y = RNG.uniform(-1, 1, (3, 80))
    grad = RNG.uniform(0.75, 1.25, (3, 1))
    tx, ty = t64(x).requires_grad_(), t64(y).requires_grad_()
    xc = tx - tx.mean(-1, keepdim=True)
    yc = ty - ty.mean(-1, keepdim=True)
    r = (xc * yc).sum(-1, keepdim=True) * torch.rsqrt((xc * xc).sum(-1, keepdim=True) + 1e-6) * torch.rsqrt(
        (yc * yc).sum(-1, keepdim=True) + 1e-6)
    r.backward(t64(grad))
    dx, dy = ref.pearson_backward(x, y, grad)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dy, ty.grad.numpy(), rtol=1e-9, atol=1e-12)


# ---------------------------------------------------------------- C5 ------


def test_gelu_tanh_matches_torch_and_limits():
    v = np.linspace(-8, 8, 101)
    np.testing.assert_allclose(ref.gelu_tanh(v), F.gelu(t64(v), approximate="tanh").numpy(), rtol=1e-14, atol=1e-15)
    assert ref.gelu_tanh(0.0) == 0.0
    assert ref.gelu_tanh(40.0) == pytest.approx(40.0) and abs(ref.gelu_tanh(-40.0)) < 1e-300


def test_ffn_matches_torch_composition():
    x = RNG.standard_normal((8, 64))
    w1 = RNG.normal(0, 1 / 8, (64, 96))
    w2 = RNG.normal(0, 1 / math.sqrt(96), (96, 64))
    out = ref.ffn_rmsnorm_gelu(x, w1, w2, 1e-6, round_h=False)
    tx = t64(x)
    a = F.rms_norm(tx, (64,), None, 1e-6)
    a = a.float().bfloat16().double()
    expect = tx + F.gelu(a @ t64(w1), approximate="tanh") @ t64(w2)
    np.testing.assert_allclose(out, expect.numpy(), rtol=1e-12, atol=1e-12)
    # round_a=False: the normalised activations stay unrounded.
    out = ref.ffn_rmsnorm_gelu(x, w1, w2, 1e-6, round_h=False, round_a=False)
    a = F.rms_norm(tx, (64,), None, 1e-6)
    expect = tx + F.gelu(a @ t64(w1), approximate="tanh") @ t64(w2)
    np.testing.assert_allclose(out, expect.numpy(), rtol=1e-12, atol=1e-12)


def test_gelu_tanh_grad_matches_autograd():
    v = RNG.uniform(-6, 6, 1000)
    tv = t64(v).requires_grad_()
    F.gelu(tv, approximate="tanh").sum().backward()
    np.testing.assert_allclose(ref.gelu_tanh_grad(v), tv.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_ffn_backward_matches_autograd():
    """Exact gradients (rounding=False) against float64 autograd of the
    forward composition, for x, W1 and W2."""
    x = RNG.standard_normal((6, 32))
    w1 = RNG.normal(0, 1 / math.sqrt(32), (32, 48))
    w2 = RNG.normal(0, 1 / math.sqrt(48), (48, 32))
    dout = RNG.standard_normal((6, 32))
    tx, tw1, tw2 = (t64(t).requires_grad_() for t in (x, w1, w2))
    a = F.rms_norm(tx, (32,), None, 1e-6)
    out = tx + F.gelu(a @ tw1, approximate="tanh") @ tw2
    out.backward(t64(dout))
    dx, dw1, dw2 = ref.ffn_rmsnorm_gelu_backward(x, w1, w2, dout, 1e-6, rounding=False)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw1, tw1.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw2, tw2.grad.numpy(), rtol=1e-10, atol=1e-12)
    # The bf16 roundings of the GPU path move the result by bf16 amounts only.
    rdx, rdw1, rdw2 = ref.ffn_rmsnorm_gelu_backward(x, w1, w2, dout, 1e-6, rounding=True)
    for got, exact in ((rdx, dx), (rdw1, dw1), (rdw2, dw2)):
        assert np.abs(got - exact).max() <= 0.05 * np.abs(exact).max()


# ------------------------------------------------------------- helpers ----


def test_bf16_rounding_matches_torch():
    v = np.concatenate([RNG.standard_normal(10000).astype(np.float32),
                        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-40, 3.0e38], dtype=np.float32)])
    bits = ref.f32_to_bf16_bits(v)
    tb = torch.from_numpy(v).bfloat16().view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(v)
    assert np.array_equal(bits[finite], tb[finite])
    assert np.isnan(ref.bf16_bits_to_f32(bits[~finite])).all()


def test_hash_lcg_known_values():
    # idx 0: 12345 >> 16 = 0 and 1013904223 >> 16 = 15470
    assert ref.hash_lcg_a(0) == 0 and ref.hash_lcg_b(0) == 15470
    # idx 1: (1103515245 + 12345) >> 16 = 16838 ; (1664525 + 1013904223) >> 16 = 15496
    assert ref.hash_lcg_a(1) == 16838 and ref.hash_lcg_b(1) == 15496
    # idx 2^20: the 64-bit product is truncated to 32 bits after the shift
    i = 1 << 20
    assert int(ref.hash_lcg_a(i)) == ((i * 1103515245 + 12345) >> 16) & 0xFFFFFFFF
    x, dy, gamma = ref.layernorm_backward_init(2, 4)
    assert x[0, 0] == np.float32(0 * (1 / 1024) - 1)
    assert gamma[1] == np.float32(0.75 + 1 * 0.015625)


def test_reference_init_restatements():
    """The init kernels of lars_momentum.cu:257-275,
    weighted_var_backward.cu:253-285 and pearson_backward.cu:289-309 at
    hand-computed indices."""
    # idx 0: (0*22695477 + 1) >> 16 = 0;  idx 1: 22695478 >> 16 = 346
    assert ref.hash_lcg_c(0) == 0 and ref.hash_lcg_c(1) == 346
    w, g, m = ref.lars_momentum_init(1, 2)
    assert w[0, 1] == np.float32((16838 & 2047) / 1024 - 1)  # 454/1024 - 1
    assert g[0, 0] == np.float32((15470 & 2047) / 1024 - 1)
    assert m[0, 1] == np.float32((346 & 2047) / 1024 - 1)
    x, wt, dy = ref.weighted_var_backward_init(1, 2)
    # base + tiny, each an fp32 operation: a & 4095 = 454 at idx 1
    expect = np.float32(np.float32(454) * np.float32(1 / 1024) - np.float32(2)) + np.float32(
        np.float32(15496 & 255) * np.float32(1e-7))
    assert x[0, 1] == expect
    assert wt[0, 0] == np.float32(0.5 + (15470 & 4095) / 4096)
    assert dy[0, 1] == np.float32((346 & 4095) / 2048 - 1)
    x, y, grad = ref.pearson_backward_init(18, 1)
    assert grad.shape == (18, 1) and grad[17, 0] == np.float32(0.75) and grad[16, 0] == np.float32(0.75 + 16 * 0.03125)


def test_gelu_tanh_pinned_to_torch_and_on_its_tails():
    """gelu_tanh / gelu_tanh_grad against torch's float64 tanh-form GELU on
    [-6, 6], and on the tails (where 1 + tanh z cancels in float64) against
    the same formula evaluated with 60-digit decimals."""
    import decimal

    v = np.linspace(-6.0, 6.0, 2001)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    tg = F.gelu(tv, approximate="tanh")
    tg.sum().backward()
    np.testing.assert_allclose(ref.gelu_tanh(v), tg.detach().numpy(), rtol=1e-13, atol=1e-15)
    # torch evaluates 1 - tanh^2 and 1 + tanh directly: absolute agreement on the tail
    np.testing.assert_allclose(ref.gelu_tanh_grad(v), tv.grad.numpy(), rtol=1e-12, atol=1e-14)

    ctx = decimal.Context(prec=60)
    c = ctx.sqrt(decimal.Decimal(2) / ctx.divide(decimal.Decimal(
        "3.14159265358979323846264338327950288419716939937510582097494"), 1))
    for x in (-7.0, -9.0, -12.0, 8.0):
        d = decimal.Decimal(x)
        z = c * (d + decimal.Decimal("0.044715") * d * d * d)
        e2 = ctx.exp(2 * z)
        tanh = (e2 - 1) / (e2 + 1)
        exact = float(decimal.Decimal("0.5") * d * (1 + tanh))
        assert ref.gelu_tanh(np.array([x]))[0] == pytest.approx(exact, rel=1e-12)
