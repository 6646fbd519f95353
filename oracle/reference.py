"""Float64 restatements of the wide-row workloads (test infrastructure only).

Each function takes numpy arrays (any float dtype; bf16 data arrives as the
float32 values of its bit patterns, see ``bf16_bits_to_f32``) and computes in
float64.  Rounding to the output dtype is left to the caller/test, except
where the workload itself rounds an intermediate (the FFN's bf16 ``h``).

How each function is pinned (tests/test_oracle.py):

* ``row_sum_max``            -- torch.sum/amax in float64; math.fsum on tiny
                                rows; NaN/inf propagation cases.
* ``layernorm_fwd``          -- F.layer_norm in float64; torch.var_mean; a
                                constant row (var = 0 -> y = beta).
* ``layernorm_backward``     -- autograd of F.layer_norm in float64.
* ``rmsnorm_fwd``            -- F.rms_norm in float64; constant-row case.
* ``rmsnorm_bwd``            -- autograd of F.rms_norm in float64 (dx, dweight).
* ``softmax_fwd``            -- torch.softmax / logsumexp / amax in float64;
                                a one-hot spike row.
* ``softmax_bwd``            -- autograd of torch.softmax in float64.
* ``softmax_logits_backward``-- autograd of torch.softmax in float64.
* ``lars_momentum``          -- closed-form special cases (zero momentum and
                                gradient; zero weight).
* ``rowwise_quant``          -- exhaustive brute force on tiny rows (the
                                argmax element quantises to +-127, the
                                zero row gives scale 0); numpy.rint ties.
* ``weighted_var_backward``  -- autograd of the weighted standardisation it
                                differentiates (agrees up to O(eps) terms).
* ``pearson_backward``       -- autograd of the Pearson correlation.
* ``ffn_rmsnorm_gelu``       -- F.rms_norm -> matmul -> F.gelu(tanh) ->
                                matmul in float64, and the GELU-tanh closed
                                form at 0 and +-large.
* ``hash_lcg_*``             -- the reference's init kernels are closed
                                integer forms; pinned by hand-computed
                                values at idx = 0, 1 and 2^20.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------- helpers --


def f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even, NaN kept quiet."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    out = np.where(nan, (u >> 16) | np.uint32(0x40), rounded)
    return out.astype(np.uint16)


def round_bf16(values: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 value (through float32), returned as float64."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(values, dtype=np.float32))).astype(np.float64)


# ----------------------------------------------------- C1: row sum / max --


def row_sum_max(x) -> tuple[np.ndarray, np.ndarray]:
    """sum and max over the last axis.

    The max is the reduction of src/workloads/rowwise_quant.cu:268-272
    (there over |x|) and dsmem_eval/workloads.py:151 (torch.amax); a NaN
    anywhere in the row makes the max NaN, as torch.amax does.
    """
    x = f64(x)
    s = x.sum(axis=-1)
    m = np.max(x, axis=-1)  # numpy max propagates NaN like torch.amax
    return s, m


# ------------------------------------------------------------- LayerNorm --


def layernorm_fwd(x, gamma, beta, eps: float = 1.0e-5):
    """Two-pass LayerNorm forward: (y, mean, rstd).

    Statistics as dsmem_eval/workloads.py:54-56 (mean, centred variance,
    rsqrt(var + eps)); the affine step is the standard y = xhat*gamma + beta.
    """
    x = f64(x)
    mean = x.mean(axis=-1, keepdims=True)
    xmu = x - mean
    var = (xmu * xmu).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = xmu * rstd * f64(gamma) + f64(beta)
    return y, mean[..., 0], rstd[..., 0]


def layernorm_backward(x, dy, gamma, eps: float = 1.0e-5):
    """dx of LayerNorm, dsmem_eval/workloads.py:53-61."""
    x, dy, gamma = f64(x), f64(dy), f64(gamma)
    mean = x.mean(axis=-1, keepdims=True)
    xmu = x - mean
    inv_std = 1.0 / np.sqrt((xmu * xmu).mean(axis=-1, keepdims=True) + eps)
    xhat = xmu * inv_std
    dyg = dy * gamma
    mean_dyg = dyg.mean(axis=-1, keepdims=True)
    mean_dyg_xhat = (dyg * xhat).mean(axis=-1, keepdims=True)
    return (dyg - mean_dyg - xhat * mean_dyg_xhat) * inv_std


# --------------------------------------------------------------- RMSNorm --


def rmsnorm_fwd(x, w, eps: float = 1.0e-6):
    """y = x * rstd * w with rstd = 1/sqrt(mean(x^2) + eps): (y, rstd).

    No reference kernel; the row sum of squares is the pattern of
    src/workloads/lars_momentum.cu:283-319 (dsmem_eval/workloads.py:139-140).
    """
    x = f64(x)
    rstd = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * rstd * f64(w), rstd[..., 0]


def rmsnorm_bwd(x, w, dy, rstd):
    """(dx, dweight) of RMSNorm given the forward's rstd.

    g = dy*w, xhat = x*rstd, dx = rstd*(g - xhat*mean(g*xhat)),
    dweight = sum over rows of dy*xhat.
    """
    x, w, dy = f64(x), f64(w), f64(dy)
    rstd = f64(rstd)[..., None]
    g = dy * w
    xhat = x * rstd
    c = (g * xhat).mean(axis=-1, keepdims=True)
    dx = rstd * (g - xhat * c)
    dw = (dy * xhat).sum(axis=0)
    return dx, dw


def rmsnorm_fwd_bwd(x, w, dy, eps: float = 1.0e-6, rstd_fp32: bool = True):
    """(y, rstd, dx, dweight) of the fused forward + backward: the forward,
    then the backward from its rstd.  rstd_fp32: the backward takes rstd
    rounded to fp32, as the fused kernel carries it (its y, dx and dweight
    all use the fp32 rstd); False keeps it in float64 (the form pinned to
    autograd)."""
    y, rstd = rmsnorm_fwd(x, w, eps)
    r = rstd.astype(np.float32) if rstd_fp32 else rstd
    y = f64(x) * f64(r)[..., None] * f64(w) if rstd_fp32 else y
    dx, dw = rmsnorm_bwd(x, w, dy, r)
    return y, rstd, dx, dw


# --------------------------------------------------------------- softmax --


def softmax_fwd(x):
    """(P, rowmax, logsumexp) of the last axis."""
    x = f64(x)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    s = e.sum(axis=-1, keepdims=True)
    return e / s, m[..., 0], (m + np.log(s))[..., 0]


def softmax_bwd(p, dy):
    """dx = P * (dy - sum(P*dy)), the backward of softmax given P."""
    p, dy = f64(p), f64(dy)
    dot = (p * dy).sum(axis=-1, keepdims=True)
    return p * (dy - dot)


def softmax_logits_backward(logits, dy):
    """Fused softmax-then-backward, dsmem_eval/workloads.py:122-125."""
    p, _, _ = softmax_fwd(logits)
    return softmax_bwd(p, dy)


# ------------------------------------------------ other reference workloads --


def lars_momentum(weight, grad, momentum):
    """(new weight, update), dsmem_eval/workloads.py:136-143."""
    w, g, m = f64(weight), f64(grad), f64(momentum)
    update = 0.9 * m + g + 0.01 * w
    wn = np.sqrt((w * w).sum(axis=-1, keepdims=True))
    un = np.sqrt((update * update).sum(axis=-1, keepdims=True))
    trust = 0.02 * wn / (un + 1.0e-6)
    return w - 1.0e-3 * trust * update, update


def rowwise_quant(x):
    """(int8 q, fp32 scale), dsmem_eval/workloads.py:150-154, for finite x.

    Computed in float32 like the reference (its inputs and scale are fp32);
    round-half-to-even as torch.round / nearbyintf
    (src/workloads/rowwise_quant.cu:239-244).  The reference's
    ``127.0 / max_abs`` is a scalar divided by a tensor, which torch
    evaluates as ``reciprocal(max_abs) * 127`` -- two fp32 roundings, not
    one correctly rounded division (the CUDA file's ``kQMax / max_abs``,
    rowwise_quant.cu:277, differs from it in about a quarter of rows) -- so
    the oracle rounds the reciprocal first.  ``scale = max_abs / 127.0`` is a
    tensor divided by a scalar: one correctly rounded division.
    """
    x = np.asarray(x, dtype=np.float32)
    max_abs = np.max(np.abs(x), axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        recip = (np.float32(1.0) / max_abs).astype(np.float32)
        inv = np.where(max_abs > 0, recip * np.float32(127.0), np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
    return q, (max_abs / np.float32(127.0)).astype(np.float32)[..., 0]


def weighted_var_backward(x, weight, dy, eps: float = 1.0e-5):
    """dsmem_eval/workloads.py:72-85 (eps 1e-5 as there; the CUDA file uses
    1e-6, src/workloads/weighted_var_backward.cu:34)."""
    x, w, dy = f64(x), f64(weight), f64(dy)
    inv_sum_w = 1.0 / (w.sum(axis=-1, keepdims=True) + eps)
    mean = (w * x).sum(axis=-1, keepdims=True) * inv_sum_w
    diff = x - mean
    variance = (w * diff * diff).sum(axis=-1, keepdims=True) * inv_sum_w
    inv_std = 1.0 / np.sqrt(variance + eps)
    sum_dy = dy.sum(axis=-1, keepdims=True)
    sum_dyc = (dy * diff).sum(axis=-1, keepdims=True)
    return inv_std * (dy - w * inv_sum_w * sum_dy - w * diff * inv_std * inv_std * inv_sum_w * sum_dyc)


def pearson_backward(x, y, grad, eps: float = 1.0e-6):
    """(dx, dy), dsmem_eval/workloads.py:96-112 (eps 1e-6 as there; the CUDA
    file uses 1e-5, src/workloads/pearson_backward.cu:34)."""
    x, y, grad = f64(x), f64(y), f64(grad)
    xc = x - x.mean(axis=-1, keepdims=True)
    yc = y - y.mean(axis=-1, keepdims=True)
    var_x = (xc * xc).sum(axis=-1, keepdims=True)
    var_y = (yc * yc).sum(axis=-1, keepdims=True)
    cov = (xc * yc).sum(axis=-1, keepdims=True)
    inv_x = 1.0 / np.sqrt(var_x + eps)
    inv_y = 1.0 / np.sqrt(var_y + eps)
    inv_xy = inv_x * inv_y
    cx = cov * inv_x**3 * inv_y
    cy = cov * inv_x * inv_y**3
    return grad * (yc * inv_xy - xc * cx), grad * (xc * inv_xy - yc * cy)


# -------------------------------------------------------------------- FFN --


def _sigmoid(a):
    """1 / (1 + e^-a) without overflow or cancellation on either side."""
    ea = np.exp(-np.abs(a))
    return np.where(a >= 0, 1.0 / (1.0 + ea), ea / (1.0 + ea))


def gelu_tanh(v):
    """0.5 v (1 + tanh z), z = sqrt(2/pi) (v + 0.044715 v^3), evaluated as
    v * sigmoid(2z) (the same function: 0.5 (1 + tanh z) = sigmoid(2z)), so
    the negative tail keeps its relative accuracy where 1 + tanh z would
    cancel in float64 (v below about -6)."""
    v = f64(v)
    return v * _sigmoid(2.0 * np.sqrt(2.0 / np.pi) * (v + 0.044715 * v**3))


def ffn_rmsnorm_gelu(x, w1, w2, eps: float = 1.0e-6, round_h: bool = True,
                     round_a: bool = True):
    """out = x + GELU_tanh(RMSNorm(x) @ W1) @ W2 (unit RMSNorm weight).

    h is rounded to bf16 as the GPU path feeds it to bf16 MFMA; the
    normalised activations a = x rstd too with round_a (the 128-tile GEMM
    scales and rounds the A tile as it stages it), while round_a=False is
    the 256-tile GEMM's arithmetic: x @ W1 on the bf16 x, the fp32 sum then
    scaled by rstd, so a is never rounded.  Accumulation is float64 here.
    """
    x = f64(x)
    rstd = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    a = round_bf16(x * rstd) if round_a else x * rstd
    h = gelu_tanh(a @ f64(w1))
    if round_h:
        h = round_bf16(h)
    return x + h @ f64(w2)


def gelu_tanh_grad(v):
    """d/dv of gelu_tanh: 0.5 (1 + tanh z) + 0.5 v (1 - tanh^2 z) dz/dv,
    z = sqrt(2/pi) (v + 0.044715 v^3); with s = sigmoid(2z) = 0.5 (1 + tanh z)
    and r = 1 - s = sigmoid(-2z), 0.5 (1 - tanh^2 z) = 2 s r, so the
    derivative is s + 2 v s r dz/dv, free of cancellation on both tails."""
    v = f64(v)
    c = np.sqrt(2.0 / np.pi)
    z2 = 2.0 * c * (v + 0.044715 * v**3)
    s, r = _sigmoid(z2), _sigmoid(-z2)
    return s + 2.0 * v * s * r * c * (1.0 + 3.0 * 0.044715 * v * v)


def ffn_rmsnorm_gelu_backward(x, w1, w2, dout, eps: float = 1.0e-6, rounding: bool = True):
    """(dx, dW1, dW2) of out = x + GELU_tanh(RMSNorm(x) @ W1) @ W2 (unit
    RMSNorm weight) for the upstream gradient dout, with W1 [d, f] and
    W2 [f, d] in the BASELINE layout; float64 arithmetic.

    rounding=True mirrors the bf16 tensors the GPU path materialises for
    bf16 MFMA: a = bf16(x rstd) (GEMM operand), u = bf16(a W1) (the saved
    pre-activation gelu' is taken at), h = bf16(gelu(u)) and du =
    bf16(dh gelu'(u)).  The RMSNorm backward uses the unrounded x rstd.
    rounding=False is the exact gradient (tests compare it with autograd).
    """
    x, w1, w2, dout = f64(x), f64(w1), f64(w2), f64(dout)
    r = round_bf16 if rounding else (lambda v: v)
    rstd = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    ahat = x * rstd
    a = r(ahat)
    u_exact = a @ w1
    u = r(u_exact)
    h = r(gelu_tanh(u_exact))
    dh = dout @ w2.T
    du = r(dh * gelu_tanh_grad(u))
    dw2 = h.T @ dout
    dw1 = a.T @ du
    da = du @ w1.T
    dx = dout + rstd * (da - ahat * (da * ahat).mean(axis=-1, keepdims=True))
    return dx, dw1, dw2


# --------------------------------------------- reference input generators --


def hash_lcg_a(idx) -> np.ndarray:
    """(idx*1103515245 + 12345) >> 16, truncated to 32 bits, as the init
    kernels of src/workloads/*.cu compute it (e.g. layernorm_backward.cu:258-259)."""
    i = np.asarray(idx, dtype=np.uint64)
    return ((i * np.uint64(1103515245) + np.uint64(12345)) >> np.uint64(16)).astype(np.uint32)


def hash_lcg_b(idx) -> np.ndarray:
    """(idx*1664525 + 1013904223) >> 16 (layernorm_backward.cu:260-261)."""
    i = np.asarray(idx, dtype=np.uint64)
    return ((i * np.uint64(1664525) + np.uint64(1013904223)) >> np.uint64(16)).astype(np.uint32)


def layernorm_backward_init(rows: int, cols: int):
    """x, dy, gamma of src/workloads/layernorm_backward.cu:253-272."""
    idx = np.arange(rows * cols, dtype=np.uint64)
    x = (hash_lcg_a(idx) & 2047).astype(np.float32) * np.float32(1.0 / 1024.0) - np.float32(1.0)
    dy = (hash_lcg_b(idx) & 2047).astype(np.float32) * np.float32(1.0 / 1024.0) - np.float32(1.0)
    col = np.arange(cols)
    gamma = np.float32(0.75) + (col % 31).astype(np.float32) * np.float32(0.015625)
    return x.reshape(rows, cols), dy.reshape(rows, cols), gamma.astype(np.float32)


def hash_lcg_c(idx) -> np.ndarray:
    """(idx*22695477 + 1) >> 16 (lars_momentum.cu:268-269)."""
    i = np.asarray(idx, dtype=np.uint64)
    return ((i * np.uint64(22695477) + np.uint64(1)) >> np.uint64(16)).astype(np.uint32)


def _grid(bits, mask: int, scale: float, offset: float) -> np.ndarray:
    return (bits & mask).astype(np.float32) * np.float32(scale) + np.float32(offset)


def lars_momentum_init(rows: int, cols: int):
    """weight, grad, momentum of src/workloads/lars_momentum.cu:257-275."""
    idx = np.arange(rows * cols, dtype=np.uint64)
    w = _grid(hash_lcg_a(idx), 2047, 1.0 / 1024.0, -1.0)
    g = _grid(hash_lcg_b(idx), 2047, 1.0 / 1024.0, -1.0)
    m = _grid(hash_lcg_c(idx), 2047, 1.0 / 1024.0, -1.0)
    return w.reshape(rows, cols), g.reshape(rows, cols), m.reshape(rows, cols)


def weighted_var_backward_init(rows: int, cols: int):
    """x, weight, dy of src/workloads/weighted_var_backward.cu:253-285."""
    idx = np.arange(rows * cols, dtype=np.uint64)
    base = _grid(hash_lcg_a(idx), 4095, 1.0 / 1024.0, -2.0)
    tiny = (hash_lcg_b(idx) & 255).astype(np.float32) * np.float32(1.0e-7)
    x = (base + tiny).astype(np.float32)
    w = np.float32(0.5) + (hash_lcg_b(idx) & 4095).astype(np.float32) * np.float32(1.0 / 4096.0)
    dy = _grid(hash_lcg_c(idx), 4095, 1.0 / 2048.0, -1.0)
    return x.reshape(rows, cols), w.astype(np.float32).reshape(rows, cols), dy.reshape(rows, cols)


def pearson_backward_init(rows: int, cols: int):
    """x, y, grad of src/workloads/pearson_backward.cu:289-309."""
    idx = np.arange(rows * cols, dtype=np.uint64)
    x = _grid(hash_lcg_a(idx), 2047, 1.0 / 1024.0, -1.0)
    y = _grid(hash_lcg_b(idx), 2047, 1.0 / 1024.0, -1.0)
    grad = np.float32(0.75) + (np.arange(rows) % 17).astype(np.float32) * np.float32(0.03125)
    return x.reshape(rows, cols), y.reshape(rows, cols), grad.astype(np.float32).reshape(rows, 1)

