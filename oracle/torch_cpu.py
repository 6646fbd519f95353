"""The reference's PyTorch path run on CPU tensors (test infrastructure only).

Used as bench.py's ``cpu_baseline`` leg: the workloads as the reference's
eager PyTorch functions compute them (dsmem_eval/workloads.py:53-154 style:
fp32 arithmetic, library reductions), on the host cores of the GPU box.  For
the BASELINE configurations without a reference function the restatement
uses the library routines BASELINE.md names (torch.sum/amax, LayerNorm on
x.float(), F.rms_norm, torch.softmax/logsumexp, GELU-tanh FFN).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def row_sum_max(x):
    return torch.sum(x, dim=-1), torch.amax(x, dim=-1)


def layernorm_fwd(x, gamma, beta, eps=1.0e-5):
    xf = x.float()
    var, mean = torch.var_mean(xf, dim=-1, unbiased=False, keepdim=True)
    rstd = torch.rsqrt(var + eps)
    y = ((xf - mean) * rstd * gamma.float() + beta.float()).to(x.dtype)
    return y, mean.squeeze(-1), rstd.squeeze(-1)


def rmsnorm_fwd(x, w, eps=1.0e-6):
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * rstd * w.float()).to(x.dtype), rstd.squeeze(-1)


def rmsnorm_bwd(x, w, dy, rstd):
    xf, dyf = x.float(), dy.float()
    r = rstd.unsqueeze(-1)
    g = dyf * w.float()
    xhat = xf * r
    c = (g * xhat).mean(dim=-1, keepdim=True)
    return (r * (g - xhat * c)).to(x.dtype), (dyf * xhat).sum(dim=0)


def softmax_fwd(x):
    m = torch.amax(x, dim=-1)
    lse = torch.logsumexp(x, dim=-1)
    return torch.softmax(x, dim=-1), m, lse


def softmax_bwd(p, dy):
    return p * (dy - (p * dy).sum(dim=-1, keepdim=True))


def layernorm_backward(x, dy, gamma):
    mean = x.mean(dim=-1, keepdim=True)
    xmu = x - mean
    inv_std = torch.rsqrt((xmu * xmu).mean(dim=-1, keepdim=True) + 1.0e-5)
    xhat = xmu * inv_std
    dyg = dy * gamma
    return (dyg - dyg.mean(dim=-1, keepdim=True) - xhat * (dyg * xhat).mean(dim=-1, keepdim=True)) * inv_std


def softmax_logits_backward(logits, dy):
    p = torch.softmax(logits, dim=-1)
    return p * (dy - (p * dy).sum(dim=-1, keepdim=True))


def rowwise_quant(x):
    """dsmem_eval/workloads.py:150-154 as written."""
    max_abs = torch.amax(torch.abs(x), dim=-1, keepdim=True)
    inv_scale = torch.where(max_abs > 0.0, 127.0 / max_abs, torch.zeros_like(max_abs))
    q = torch.clamp(torch.round(x * inv_scale), -127.0, 127.0).to(torch.int8)
    return q, (max_abs / 127.0).squeeze(-1)


def lars_momentum(weight, grad, momentum):
    """dsmem_eval/workloads.py:136-143 as written."""
    update = 0.9 * momentum + grad + 0.01 * weight
    weight_norm = torch.sqrt((weight * weight).sum(dim=-1, keepdim=True))
    update_norm = torch.sqrt((update * update).sum(dim=-1, keepdim=True))
    trust = 0.02 * weight_norm / (update_norm + 1.0e-6)
    return weight - 1.0e-3 * trust * update, update


def weighted_var_backward(x, weight, dy):
    """dsmem_eval/workloads.py:72-85 as written."""
    inv_sum_w = 1.0 / (weight.sum(dim=-1, keepdim=True) + 1.0e-5)
    mean = (weight * x).sum(dim=-1, keepdim=True) * inv_sum_w
    diff = x - mean
    variance = (weight * diff * diff).sum(dim=-1, keepdim=True) * inv_sum_w
    inv_std = torch.rsqrt(variance + 1.0e-5)
    sum_dy = dy.sum(dim=-1, keepdim=True)
    sum_dyc = (dy * diff).sum(dim=-1, keepdim=True)
    return inv_std * (dy - weight * inv_sum_w * sum_dy
                      - weight * diff * inv_std * inv_std * inv_sum_w * sum_dyc)


def pearson_backward(x, y, grad):
    """dsmem_eval/workloads.py:96-112 as written."""
    xc = x - x.mean(dim=-1, keepdim=True)
    yc = y - y.mean(dim=-1, keepdim=True)
    inv_x = torch.rsqrt((xc * xc).sum(dim=-1, keepdim=True) + 1.0e-6)
    inv_y = torch.rsqrt((yc * yc).sum(dim=-1, keepdim=True) + 1.0e-6)
    cov = (xc * yc).sum(dim=-1, keepdim=True)
    inv_xy = inv_x * inv_y
    return (grad * (yc * inv_xy - xc * cov * inv_x * inv_x * inv_x * inv_y),
            grad * (xc * inv_xy - yc * cov * inv_x * inv_y * inv_y * inv_y))


def ffn(x, w1, w2, eps=1.0e-6):
    a = F.rms_norm(x.float(), (x.shape[-1],), None, eps).to(x.dtype)
    h = F.gelu(a @ w1, approximate="tanh")
    return (x.float() + (h @ w2).float()).to(x.dtype)


def ffn_backward(x, w1, w2, dout, eps=1.0e-6):
    """Autograd of ffn() in the inputs' dtype: (dx, dW1, dW2)."""
    x = x.detach().requires_grad_()
    w1 = w1.detach().requires_grad_()
    w2 = w2.detach().requires_grad_()
    a = F.rms_norm(x.float(), (x.shape[-1],), None, eps).to(x.dtype)
    out = x + F.gelu(a @ w1, approximate="tanh") @ w2
    out.backward(dout)
    return x.grad, w1.grad, w2.grad


def ffn_backward_saved(x, w1, w2, dout, eps=1.0e-6):
    """The autograd graph of ffn() built once, its activations kept: returns
    a function that runs only the backward pass, (dx, dW1, dW2)."""
    x = x.detach().requires_grad_()
    w1 = w1.detach().requires_grad_()
    w2 = w2.detach().requires_grad_()
    a = F.rms_norm(x.float(), (x.shape[-1],), None, eps).to(x.dtype)
    out = x + F.gelu(a @ w1, approximate="tanh") @ w2
    return lambda: torch.autograd.grad(out, (x, w1, w2), dout, retain_graph=True)


# name -> (function, which BASELINE inputs it takes)
FUNCTIONS = {
    "row_sum_max": row_sum_max,
    "layernorm_fwd": layernorm_fwd,
    "rmsnorm_fwd": lambda x, w, dy: rmsnorm_fwd(x, w),
    "rmsnorm_bwd": lambda x, w, dy: rmsnorm_bwd(x, w, dy, rmsnorm_fwd(x, w)[1]),
    "rmsnorm_fwd_bwd": lambda x, w, dy: (lambda f: (f, rmsnorm_bwd(x, w, dy, f[1])))(
        rmsnorm_fwd(x, w)),
    "softmax_fwd": lambda x, dy: softmax_fwd(x),
    "softmax_bwd": lambda x, dy: softmax_bwd(torch.softmax(x, dim=-1), dy),
    "layernorm_backward": layernorm_backward,
    "layernorm_backward_bf16": lambda x, dy, g: layernorm_backward(
        x.float(), dy.float(), g.float()).to(x.dtype),
    "softmax_logits_backward": softmax_logits_backward,
    "rowwise_quant": rowwise_quant,
    "lars_momentum": lars_momentum,
    "weighted_var_backward": weighted_var_backward,
    "pearson_backward": pearson_backward,
    "ffn": ffn,
    "ffn_baseline_layout": ffn,
    "ffn_backward": ffn_backward,
    "ffn_backward_baseline_layout": ffn_backward,
    # Builds the graph and returns the backward-only call (bench.py times
    # that call).
    "ffn_backward_saved": ffn_backward_saved,
}
