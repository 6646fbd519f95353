"""GPU parity of credit_ffn_rmsnorm_gelu_bf16 (C5), its [in, out]-weight form
credit_ffn_rmsnorm_gelu_kn_bf16 and credit_transpose_bf16.

out = x + GELU_tanh(RMSNorm(x) @ W1) @ W2 against the float64 oracle
(oracle.reference.ffn_rmsnorm_gelu, which rounds the normalised activations
and h to bf16 as the MFMA path feeds them).  Tolerance: bf16 output within
rtol 1e-2 / atol 1e-2.  The small shapes also pin the
MFMA operand/accumulator lane layout: a wrong row/column mapping scrambles
every output.  At the full C5 shape the oracle checks a sample of rows
(each row of out depends only on the same row of x), and every element is
checked against a float32 restatement on the GPU (torch_fp32_ffn), itself
held to the oracle on sampled rows."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS, make_ffn_inputs
from oracle import reference as ref

pytestmark = pytest.mark.gpu

EPS = 1.0e-6
BF16 = dict(rtol=1e-2, atol=1e-2)


def make(rows, d, f, seed):
    g = torch.Generator().manual_seed(seed)
    return make_ffn_inputs(rows, d, g, ffn_dim=f)


def run_ffn(x, w1, w2, gpu):
    xs = x.to(gpu)
    w1t = hip_lib.linear_layout(w1.to(gpu))
    w2t = hip_lib.linear_layout(w2.to(gpu))
    out = torch.full_like(xs, float("nan"))
    hip_lib.ffn(xs, w1t, w2t, out, EPS, hip_lib.make_cfg())
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def run_ffn_in_out(x, w1, w2, gpu):
    """The BASELINE's [in, out] weights (W1 [d, f], W2 [f, d]) passed as they
    are: credit_ffn_rmsnorm_gelu_kn_bf16."""
    xs = x.to(gpu)
    out = torch.full_like(xs, float("nan"))
    hip_lib.ffn(xs, w1.to(gpu), w2.to(gpu), out, EPS, hip_lib.make_cfg(), layout="in_out")
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle(x, w1, w2, rows=None, round_a=True):
    xs = x.float().numpy() if rows is None else x[rows].float().numpy()
    return ref.ffn_rmsnorm_gelu(xs, w1.float().numpy(), w2.float().numpy(), EPS,
                                round_a=round_a)


# (64, 128) and (256, 1024) take the 16-byte tile path, the rest the element path.
@pytest.mark.parametrize("shape", [(64, 96), (128, 200), (3, 5), (257, 130), (64, 128),
                                   (256, 1024)])
def test_transpose_is_exact(gpu, shape):
    src = torch.randn(shape, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    dst = torch.empty(shape[1], shape[0], dtype=torch.bfloat16, device=gpu)
    hip_lib.transpose(src.to(gpu), dst)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src.t().contiguous())


# The first four take the 128-tile kernels; the rest run GEMM1 (and where
# d allows, GEMM2) on the 256-tile direct-to-LDS kernel (M and N multiples
# of 256, K of 128, tile count a multiple of 8).  (512, 128, 1024) gives it
# the shortest K (two 64-wide steps), (2048, 384, 256) an odd number of
# step pairs (six steps), (4096, 256, 4608) GEMM1 288 tiles: more than one
# workgroup per CU, so a second, partial wave of tiles.
@pytest.mark.parametrize("rows,d,f", [(128, 128, 128), (128, 256, 384), (256, 128, 512),
                                      (384, 512, 256), (512, 1024, 1024), (256, 2048, 2048),
                                      (1024, 512, 4096), (512, 128, 1024), (2048, 384, 256),
                                      (4096, 256, 4608)])
def test_ffn_small_shapes(gpu, rows, d, f):
    print(f"ffn rows={rows} d={d} f={f}", flush=True)
    x, w1, w2 = make(rows, d, f, seed=rows + d + f)
    np.testing.assert_allclose(run_ffn(x, w1, w2, gpu), oracle(x, w1, w2), **BF16)


@pytest.mark.parametrize("rows,d,f", [(128, 128, 128), (128, 256, 384), (384, 512, 256),
                                      (512, 1024, 1024), (1024, 512, 4096), (512, 128, 1024),
                                      (2048, 384, 256), (4096, 256, 4608)])
def test_ffn_in_out_layout_is_bit_identical(gpu, rows, d, f):
    """The [in, out] weight path feeds every MFMA the same operand values in
    the same lanes as the nn.Linear path (its B fragments come from
    transposing LDS reads of [K, N] tiles), so the outputs agree bit for
    bit; the first three shapes take the 128-tile kernels (B staged through
    registers), the rest the 256-tile ones, (2048, 384, 256) with GEMM2 on
    the 128-tile kernel (d = 384)."""
    print(f"ffn in_out rows={rows} d={d} f={f}", flush=True)
    x, w1, w2 = make(rows, d, f, seed=rows + d + f + 1)
    got = run_ffn_in_out(x, w1, w2, gpu)
    assert np.array_equal(got, run_ffn(x, w1, w2, gpu))
    np.testing.assert_allclose(got, oracle(x, w1, w2), **BF16)


@pytest.mark.parametrize("rows,d", [(128, 256), (2048, 256)])
def test_ffn_in_out_structured_inputs(gpu, rows, d):
    """Permutation weights on the [in, out] path: out = x + GELU(2 a[:, p])
    [:, q], so a column or K-row of the [K, N] tile read from the wrong LDS
    position (swizzle, transposing-read lane order, stage pitch) moves
    values to the wrong output column.  Each output carries one a value
    straight through GELU, so the oracle follows the kernel's arithmetic
    for a: rounded to bf16 on the 128-tile path (rows 128), unrounded on the
    256-tile path (rows 2048, both GEMMs), where the fp32 sum is scaled by
    rstd."""
    g = torch.Generator().manual_seed(5)
    p = torch.randperm(d, generator=g)
    q = torch.randperm(d, generator=g)
    x = (torch.arange(rows * d, dtype=torch.float32).reshape(rows, d) % 11 - 5).to(torch.bfloat16)
    w1 = torch.zeros(d, d)
    w1[p, torch.arange(d)] = 2.0   # h[:, j] = GELU(2 a[:, p[j]])
    w2 = torch.zeros(d, d)
    w2[torch.arange(d), q] = 1.0   # out[:, q[j]] += h[:, j]
    w1, w2 = w1.to(torch.bfloat16), w2.to(torch.bfloat16)
    np.testing.assert_allclose(run_ffn_in_out(x, w1, w2, gpu),
                               oracle(x, w1, w2, round_a=rows < 2048), **BF16)


@pytest.mark.parametrize("rows,d", [(128, 256), (2048, 256)])
def test_ffn_structured_inputs_pin_layout(gpu, rows, d):
    """Identity-like weights make each output element depend on one input
    element, so any transposed or shifted fragment mapping (or a wrong LDS
    swizzle / direct-to-LDS lane placement) fails.  (2048, 256) takes the
    256-tile kernels."""
    f = d
    x = (torch.arange(rows * d, dtype=torch.float32).reshape(rows, d) % 7 - 3).to(torch.bfloat16)
    w1 = torch.eye(d, dtype=torch.bfloat16) * 2
    w2 = torch.eye(d, dtype=torch.bfloat16)
    out = run_ffn(x, w1, w2, gpu)
    np.testing.assert_allclose(out, oracle(x, w1, w2), **BF16)


@pytest.mark.parametrize("rows", [128, 2048])
def test_ffn_gelu_negative_tail(gpu, rows):
    """GELU far out on its negative tail, where 0.5 (1 + tanh z) is a tiny
    sigmoid and 1 - r would cancel: x = 1 (a = x rstd = 1), W1 = -diag(c)
    with c from 3 to 9 (h = GELU(-c) from -4e-3 down to -1e-28) and W2 =
    diag(2 / |GELU(-c)|), so out = 1 + h * 2 / |h| = -1 where h keeps its
    relative accuracy and 1 where it was flushed to zero.  rows 128 takes the
    128-tile kernels, 2048 the 256-tile ones."""
    d = 256
    c = np.linspace(3.0, 9.0, d)
    w1 = torch.from_numpy(-np.diag(c)).to(torch.bfloat16)
    cb = -w1.float().numpy().diagonal().astype(np.float64)  # c as bf16 holds it
    g = ref.gelu_tanh(-cb)
    w2 = torch.from_numpy(np.diag(2.0 / np.abs(g))).to(torch.bfloat16)
    x = torch.ones(rows, d, dtype=torch.bfloat16)
    out = run_ffn(x, w1, w2, gpu)
    expect = oracle(x, w1, w2)
    assert np.all(np.abs(expect + 1.0) < 2e-2)  # the oracle itself sees h
    np.testing.assert_allclose(out, expect, **BF16)


def test_ffn_rejects_unsupported_shapes(gpu):
    x, w1, w2 = make(100, 128, 128, seed=3)
    with pytest.raises(hip_lib.CreditError) as err:
        run_ffn(x, w1, w2, gpu)
    assert err.value.status == -4


def test_ffn_full_config_sampled_rows(gpu):
    """BASELINE C5: x [4096, 8192], W1 [8192, 28672], W2 [28672, 8192]; 48
    rows (spread over all row tiles) against the float64 oracle."""
    x, w1, w2 = WORKLOADS["ffn"].make_inputs()
    out = run_ffn(x, w1, w2, gpu)
    rows = np.linspace(0, x.shape[0] - 1, 48).astype(int)
    # The 256-tile arithmetic: rstd applied to the fp32 accumulator (round_a=False).
    np.testing.assert_allclose(out[rows], oracle(x, w1, w2, rows, round_a=False), **BF16)
    assert np.isfinite(out).all()


def torch_fp32_ffn(x, w1, w2, gpu):
    """The 256-tile path's arithmetic in float32 on the GPU (W1 [d, f], W2 [f,
    d]): the fp32 product x @ W1 scaled by rstd (the normalised input is never
    rounded), h = bf16(GELU_tanh(u)), out = x + h @ W2, as a float32 tensor on
    the device.  Full-precision float32 products (no reduced-precision modes)."""
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        X = x.to(gpu).float()
        rstd = torch.rsqrt((X * X).mean(dim=1, keepdim=True) + EPS)
        u = (X @ w1.to(gpu).float()) * rstd
        h = torch.nn.functional.gelu(u, approximate="tanh").to(torch.bfloat16).float()
        del u
        return X + h @ w2.to(gpu).float()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev


@pytest.mark.parametrize("layout", ["linear", "in_out"])
def test_ffn_full_config_every_element(gpu, layout):
    """BASELINE C5, every element of out against torch_fp32_ffn, itself
    checked against the float64 oracle on 8 sampled rows (to a tenth of the
    tolerance): 33.5M outputs, all within rtol 1e-2 / atol 1e-2."""
    x, w1, w2 = WORKLOADS["ffn" if layout == "linear" else "ffn_baseline_layout"].make_inputs()
    print(f"ffn C5 every element, {layout} weights", flush=True)
    out = run_ffn(x, w1, w2, gpu) if layout == "linear" else run_ffn_in_out(x, w1, w2, gpu)
    expect = torch_fp32_ffn(x, w1, w2, gpu)
    rows = np.array([0, 1, 1000, 2047, 2048, 3333, 4094, 4095])
    np.testing.assert_allclose(expect[rows].cpu().numpy(),
                               oracle(x, w1, w2, rows, round_a=False), rtol=1e-3, atol=1e-3)
    got = torch.from_numpy(out).to(gpu)
    excess = (got - expect).abs() - (1e-2 * expect.abs() + 1e-2)
    worst = int(excess.argmax())
    assert float(excess.max()) <= 0, (
        f"max excess {float(excess.max()):.3e} at {np.unravel_index(worst, out.shape)}")
    assert bool(torch.isfinite(got).all())


def test_ffn_in_out_full_config_sampled_rows(gpu):
    """BASELINE C5 with W1 [8192, 28672] and W2 [28672, 8192] passed as the
    BASELINE gives them: 48 sampled rows against the float64 oracle."""
    x, w1, w2 = WORKLOADS["ffn_baseline_layout"].make_inputs()
    out = run_ffn_in_out(x, w1, w2, gpu)
    rows = np.linspace(0, x.shape[0] - 1, 48).astype(int)
    # The 256-tile arithmetic: rstd applied to the fp32 accumulator (round_a=False).
    np.testing.assert_allclose(out[rows], oracle(x, w1, w2, rows, round_a=False), **BF16)
    assert np.isfinite(out).all()
