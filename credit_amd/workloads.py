"""Workload registry: shapes, seeded inputs, traffic and tolerances.

Mirrors the reference's ``WorkloadSpec`` registry
(dsmem_eval/workloads.py:16-37,157-212) for the MI355X build.  Two families:

* the BASELINE configurations C1-C5 (row sum/max, LayerNorm forward,
  RMSNorm forward/backward, online softmax forward/backward, norm-fused
  FFN), which have no reference kernel; and
* the reference's own wide-row workloads (LayerNorm backward,
  softmax-logits backward, ...), with the input ranges, eps and tolerances of
  dsmem_eval/workloads.py.

Inputs come from a seeded CPU ``torch.Generator`` (CPU and ROCm generator
streams differ, so generating on the CPU and copying keeps the GPU run, the
oracle and the CPU baseline on identical data).  The reference seeds a CUDA
generator with 1234 + cols (dsmem_eval/runner.py:358); the BASELINE
configurations use seed 0.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

import torch

TensorTuple = tuple[torch.Tensor, ...]


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    label: str
    category: str
    rows: int
    cols: int
    input_factory: Callable[[int, int, torch.Generator], TensorTuple]
    output_names: tuple[str, ...]
    # Algorithmic (compulsory) HBM bytes of one call at (rows, cols): every
    # input read once, every output written once.  The roofline numerator.
    algorithmic_bytes: Callable[[int, int], int]
    # Per-output (atol, rtol); None means bit-exact.
    tolerances: tuple[tuple[float, float] | None, ...]
    seed: int = 0
    # Cost-model metadata (dsmem_eval/workload_metadata.py:6-35): HBM bytes
    # per element of this build's READ (no-staging) variant, the re-read share
    # staging removes, bytes staged on chip per element, partials exchanged
    # per split stage.
    modeled_bytes_per_element: float = 0.0
    reread_bytes_per_element: float = 0.0
    staged_bytes_per_element: int = 0
    reductions_per_stage: tuple[int, ...] = field(default_factory=tuple)
    # Widest row the STAGED (no-split, row held on chip) variant takes; 0 when
    # the operation has no split variant.  Wider rows need SPLIT or READ.
    staged_max_cols: int = 0
    # HBM read:write byte mix of one call, as whole streams (row_sum_max 1:0,
    # a norm forward 1:1, a backward reading x and dy for dx 2:1, ...): the
    # mix of the stream ceiling the kernel's rate is compared with.  (0, 0)
    # for compute-bound work.
    stream_mix: tuple[int, int] = (0, 0)
    # Row-steps by which this build's SPLIT kernel publishes a row's partial
    # ahead of waiting for its total (the group pipelines' DEPTH: data waves
    # publish row i+DEPTH and finish row i while a communication wave polls),
    # 0 for the barrier-synchronised slice kernels; an int, or a function of
    # (cols, split) where the split factor decides which kernel runs.  The
    # cost model hides that much of the exchange behind the stream.
    split_pipeline_depth: int | Callable[[int, int], int] = 0

    @property
    def barrier_count(self) -> int:
        """One arrival barrier per reduction stage (the reference counts two
        cluster.sync per stage, dsmem_eval/workloads.py:31-33)."""
        return len(self.reductions_per_stage)

    @property
    def partial_count(self) -> int:
        return sum(self.reductions_per_stage)

    def make_inputs(self, rows: int | None = None, cols: int | None = None, seed: int | None = None,
                    device: str | torch.device = "cpu") -> TensorTuple:
        g = torch.Generator(device="cpu")
        g.manual_seed(self.seed if seed is None else seed)
        tensors = self.input_factory(rows or self.rows, cols or self.cols, g)
        if torch.device(device).type == "cpu":
            return tensors
        return tuple(t.to(device) for t in tensors)


# ----------------------------------------------------------- factories ----


def _uniform(shape, low, high, g):
    return torch.empty(shape, dtype=torch.float32).uniform_(low, high, generator=g)


def _normal(shape, mean, std, g, dtype=torch.float32):
    t = torch.randn(shape, generator=g, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t.to(dtype)


def make_row_sum_max_inputs(rows, cols, g):
    return (_uniform((rows, cols), -1.0, 1.0, g),)


def make_layernorm_fwd_inputs(rows, cols, g):
    return (
        _normal((rows, cols), 0.0, 1.0, g, torch.bfloat16),
        _normal((cols,), 1.0, 0.02, g, torch.bfloat16),
        _normal((cols,), 0.0, 0.02, g, torch.bfloat16),
    )


def make_rmsnorm_inputs(rows, cols, g):
    return (
        _normal((rows, cols), 0.0, 1.0, g, torch.bfloat16),
        _normal((cols,), 1.0, 0.02, g, torch.bfloat16),
        _normal((rows, cols), 0.0, 1.0, g, torch.bfloat16),
    )


def make_softmax_inputs(rows, cols, g):
    """x ~ N(0, std 4) with 1% of entries set to +20; dy ~ N(0, 1).
    Draw order: x, dy, then the mask."""
    x = _normal((rows, cols), 0.0, 4.0, g)
    dy = _normal((rows, cols), 0.0, 1.0, g)
    mask = torch.rand((rows, cols), generator=g) < 0.01
    x[mask] = 20.0
    return x, dy


def make_ffn_inputs(rows, cols, g, ffn_dim: int = 28672):
    d = cols
    return (
        _normal((rows, d), 0.0, 1.0, g, torch.bfloat16),
        _normal((d, ffn_dim), 0.0, 1.0 / math.sqrt(d), g, torch.bfloat16),
        _normal((ffn_dim, d), 0.0, 1.0 / math.sqrt(ffn_dim), g, torch.bfloat16),
    )


def make_ffn_backward_inputs(rows, cols, g, ffn_dim: int = 28672):
    """The forward's x, W1, W2, then the upstream gradient dout ~ N(0, 1)."""
    x, w1, w2 = make_ffn_inputs(rows, cols, g, ffn_dim)
    return x, w1, w2, _normal((rows, cols), 0.0, 1.0, g, torch.bfloat16)


# Reference workloads: input ranges of dsmem_eval/workloads.py:45-50,115-119.


def make_layernorm_backward_inputs(rows, cols, g):
    return (
        _uniform((rows, cols), -1.0, 1.0, g),
        _uniform((rows, cols), -1.0, 1.0, g),
        _uniform((cols,), 0.75, 1.25, g),
    )


def make_layernorm_backward_bf16_inputs(rows, cols, g):
    return tuple(t.to(torch.bfloat16) for t in make_layernorm_backward_inputs(rows, cols, g))


def make_softmax_logits_inputs(rows, cols, g):
    return (
        _uniform((rows, cols), -4.0, 4.0, g),
        _uniform((rows, cols), -1.0, 1.0, g),
    )


def make_quant_inputs(rows, cols, g):
    return (_uniform((rows, cols), -1.0, 1.0, g),)


def make_lars_inputs(rows, cols, g):
    """weight, grad, momentum ~ U(-1, 1) (dsmem_eval/workloads.py:128-133)."""
    return tuple(_uniform((rows, cols), -1.0, 1.0, g) for _ in range(3))


def make_weighted_var_inputs(rows, cols, g):
    """x ~ U(-2, 2), weight ~ U(0.5, 1.5), dy ~ U(-1, 1)
    (dsmem_eval/workloads.py:64-69)."""
    return (
        _uniform((rows, cols), -2.0, 2.0, g),
        _uniform((rows, cols), 0.5, 1.5, g),
        _uniform((rows, cols), -1.0, 1.0, g),
    )


def make_pearson_inputs(rows, cols, g):
    """x, y ~ U(-1, 1), grad ~ U(0.75, 1.25) per row
    (dsmem_eval/workloads.py:88-93)."""
    return (
        _uniform((rows, cols), -1.0, 1.0, g),
        _uniform((rows, cols), -1.0, 1.0, g),
        _uniform((rows, 1), 0.75, 1.25, g),
    )


# -------------------------------------------------------------- registry --

FP32_TOL = (1.0e-6, 1.0e-5)
BF16_TOL = (1.0e-2, 1.0e-2)

def _member_vectors(cols: int, split: int, elems: int) -> int:
    """Vectors (16 bytes, `elems` elements each) per member of a P-way
    split, as the library's planners divide a row (ceil(nvec / P))."""
    nvec = cols // elems
    return -(-nvec // max(split, 1))


def _rmsnorm_fwd_depth(cols: int, split: int) -> int:
    """csrc/rmsnorm.hip fwd_takes_group: members of 1025-2048 vectors (at
    most 32) run the forward group pipeline (DEPTH 4); others the slice
    kernel."""
    chunk = _member_vectors(cols, split, 8)
    members = -(-(cols // 8) // chunk)
    return 4 if 1024 < chunk <= 2048 and members <= 32 else 0


def _softmax_fwd_depth(cols: int, split: int) -> int:
    """csrc/softmax.hip kFwdGroup: the 512-lane 8-vector shape (members of
    3841-4096 vectors) parks rows and publishes 4 steps ahead; the other
    group shapes 2."""
    return 4 if _member_vectors(cols, split, 4) > 3840 else 2


def _softmax_bwd_depth(cols: int, split: int) -> int:
    """csrc/softmax.hip kBwdGroup: the 512-lane 4-vector shape (members of
    1025-2048 vectors) parks rows and publishes 4 steps ahead; the others 2."""
    return 4 if _member_vectors(cols, split, 4) > 1024 else 2


def _layernorm_bwd_bf16_depth(cols: int, split: int) -> int:
    """csrc/lnbwd.hip: SPLIT of at most 16 members of at most 1024 vectors
    runs the bf16 group pipeline (DEPTH 4); others the slice kernel."""
    return 4 if split <= 16 and _member_vectors(cols, split, 8) <= 1024 else 0


WORKLOADS: dict[str, WorkloadSpec] = {
    "row_sum_max": WorkloadSpec(
        name="row_sum_max",
        label="Row-wise sum + max",
        category="reduction",
        rows=1024,
        cols=65536,
        input_factory=make_row_sum_max_inputs,
        output_names=("sum", "max"),
        algorithmic_bytes=lambda r, c: 4 * r * c + 8 * r,
        tolerances=(FP32_TOL, None),
        modeled_bytes_per_element=4.0,
        reread_bytes_per_element=0.0,
        staged_bytes_per_element=0,
        reductions_per_stage=(2,),
        staged_max_cols=1 << 30,
        stream_mix=(1, 0),
    ),
    "layernorm_fwd": WorkloadSpec(
        name="layernorm_fwd",
        label="LayerNorm forward (bf16)",
        category="normalization",
        rows=2048,
        cols=32768,
        input_factory=make_layernorm_fwd_inputs,
        output_names=("y", "mean", "rstd"),
        algorithmic_bytes=lambda r, c: 2 * r * c + 2 * r * c + 4 * c + 8 * r,
        tolerances=(BF16_TOL, FP32_TOL, FP32_TOL),
        modeled_bytes_per_element=8.0,  # READ: x three times (sum, deviations, output) + y
        reread_bytes_per_element=4.0,   # the second and third reads of x
        staged_bytes_per_element=2,
        reductions_per_stage=(2,),      # SPLIT: one stage of (sum, sum of squares)
        staged_max_cols=65536,
        stream_mix=(1, 1),
    ),
    "rmsnorm_fwd": WorkloadSpec(
        name="rmsnorm_fwd",
        label="RMSNorm forward (bf16)",
        category="normalization",
        rows=1024,
        cols=131072,
        input_factory=make_rmsnorm_inputs,
        output_names=("y", "rstd"),
        algorithmic_bytes=lambda r, c: 2 * r * c + 2 * c + 2 * r * c + 4 * r,
        tolerances=(BF16_TOL, FP32_TOL),
        modeled_bytes_per_element=6.0,
        reread_bytes_per_element=2.0,
        staged_bytes_per_element=2,
        reductions_per_stage=(1,),
        staged_max_cols=65536,
        stream_mix=(1, 1),
        split_pipeline_depth=_rmsnorm_fwd_depth,
    ),
    "rmsnorm_bwd": WorkloadSpec(
        name="rmsnorm_bwd",
        label="RMSNorm backward (bf16, fp32 dweight)",
        category="normalization",
        rows=1024,
        cols=131072,
        input_factory=make_rmsnorm_inputs,
        output_names=("dx", "dweight"),
        algorithmic_bytes=lambda r, c: 2 * r * c * 2 + 2 * c + 4 * r + 2 * r * c + 4 * c,
        tolerances=(BF16_TOL, FP32_TOL),
        modeled_bytes_per_element=10.0,
        reread_bytes_per_element=4.0,
        staged_bytes_per_element=4,
        reductions_per_stage=(1,),
        staged_max_cols=8192,
        split_pipeline_depth=4,
        stream_mix=(2, 1),
    ),
    # C3's forward and backward in one call (credit_rmsnorm_fwd_bwd_bf16):
    # x, dy, w in; y, rstd, dx, dweight out.
    "rmsnorm_fwd_bwd": WorkloadSpec(
        name="rmsnorm_fwd_bwd",
        label="RMSNorm forward + backward fused (bf16)",
        category="normalization",
        rows=1024,
        cols=131072,
        input_factory=make_rmsnorm_inputs,
        output_names=("y", "rstd", "dx", "dweight"),
        algorithmic_bytes=lambda r, c: 2 * r * c * 4 + 2 * c + 4 * c + 4 * r,
        tolerances=(BF16_TOL, FP32_TOL, BF16_TOL, FP32_TOL),
        stream_mix=(2, 2),
    ),
    "softmax_fwd": WorkloadSpec(
        name="softmax_fwd",
        label="Online softmax forward (fp32)",
        category="softmax",
        rows=512,
        cols=262144,
        input_factory=make_softmax_inputs,
        output_names=("p", "max", "lse"),
        algorithmic_bytes=lambda r, c: 4 * r * c * 2 + 8 * r,
        tolerances=(FP32_TOL, None, FP32_TOL),
        modeled_bytes_per_element=12.0,
        reread_bytes_per_element=4.0,
        staged_bytes_per_element=4,
        reductions_per_stage=(2,),
        staged_max_cols=65536,
        split_pipeline_depth=_softmax_fwd_depth,
        stream_mix=(1, 1),
    ),
    "softmax_bwd": WorkloadSpec(
        name="softmax_bwd",
        label="Softmax backward (fp32)",
        category="softmax",
        rows=512,
        cols=262144,
        input_factory=make_softmax_inputs,
        output_names=("dx",),
        algorithmic_bytes=lambda r, c: 4 * r * c * 3,
        tolerances=(FP32_TOL,),
        modeled_bytes_per_element=20.0,
        reread_bytes_per_element=8.0,
        staged_bytes_per_element=8,
        reductions_per_stage=(1,),
        staged_max_cols=32768,
        split_pipeline_depth=_softmax_bwd_depth,
        stream_mix=(2, 1),
    ),
    "ffn": WorkloadSpec(
        name="ffn",
        label="Norm-fused FFN (bf16 MFMA)",
        category="gemm",
        rows=4096,
        cols=8192,
        input_factory=make_ffn_inputs,
        output_names=("out",),
        algorithmic_bytes=lambda r, c: 2 * (r * c * 2 + 2 * c * 28672),
        tolerances=(BF16_TOL,),
    ),
    # C5 again, with the weights in the BASELINE's own [in, out] layout
    # (W1 [d, f], W2 [f, d]) handed to the library as they are.
    "ffn_baseline_layout": WorkloadSpec(
        name="ffn_baseline_layout",
        label="Norm-fused FFN, [in, out] weights (bf16 MFMA)",
        category="gemm",
        rows=4096,
        cols=8192,
        input_factory=make_ffn_inputs,
        output_names=("out",),
        algorithmic_bytes=lambda r, c: 2 * (r * c * 2 + 2 * c * 28672),
        tolerances=(BF16_TOL,),
    ),
    # The "backward of the fused FFN" next row: dx, dW1, dW2 for dout.
    "ffn_backward": WorkloadSpec(
        name="ffn_backward",
        label="Norm-fused FFN backward (bf16 MFMA)",
        category="gemm",
        rows=4096,
        cols=8192,
        input_factory=make_ffn_backward_inputs,
        output_names=("dx", "dw1", "dw2"),
        algorithmic_bytes=lambda r, c: 2 * (3 * r * c + 4 * c * 28672),
        tolerances=(BF16_TOL, BF16_TOL, BF16_TOL),
    ),
    # The same gradients for the BASELINE's own [in, out] weights (W1 [d, f],
    # W2 [f, d]), read as they are; dW1 [d, f] and dW2 [f, d] come back in
    # that layout.
    "ffn_backward_baseline_layout": WorkloadSpec(
        name="ffn_backward_baseline_layout",
        label="Norm-fused FFN backward, [in, out] weights (bf16 MFMA)",
        category="gemm",
        rows=4096,
        cols=8192,
        input_factory=make_ffn_backward_inputs,
        output_names=("dx", "dw1", "dw2"),
        algorithmic_bytes=lambda r, c: 2 * (3 * r * c + 4 * c * 28672),
        tolerances=(BF16_TOL, BF16_TOL, BF16_TOL),
    ),
    # The same gradients from the training forward's saved rstd, u and h
    # (no recompute GEMM).
    "ffn_backward_saved": WorkloadSpec(
        name="ffn_backward_saved",
        label="Norm-fused FFN backward from saved activations (bf16 MFMA)",
        category="gemm",
        rows=4096,
        cols=8192,
        input_factory=make_ffn_backward_inputs,
        output_names=("dx", "dw1", "dw2"),
        algorithmic_bytes=lambda r, c: 2 * (3 * r * c + 4 * c * 28672),
        tolerances=(BF16_TOL, BF16_TOL, BF16_TOL),
    ),
    # Reference workloads (dsmem_eval/workloads.py:157-212).
    "layernorm_backward": WorkloadSpec(
        name="layernorm_backward",
        label="LayerNorm backward",
        category="normalization",
        rows=2048,
        cols=65536,
        input_factory=make_layernorm_backward_inputs,
        output_names=("dx",),
        algorithmic_bytes=lambda r, c: 4 * r * c * 3 + 4 * c,
        tolerances=((2.0e-2, 2.0e-2),),
        seed=1234,
        modeled_bytes_per_element=24.0,
        reread_bytes_per_element=12.0,
        staged_bytes_per_element=4,
        reductions_per_stage=(2, 2),
        staged_max_cols=32768,
        stream_mix=(2, 1),
    ),
    "layernorm_backward_bf16": WorkloadSpec(
        name="layernorm_backward_bf16",
        label="LayerNorm backward (bf16)",
        category="normalization",
        rows=2048,
        cols=65536,
        input_factory=make_layernorm_backward_bf16_inputs,
        output_names=("dx",),
        algorithmic_bytes=lambda r, c: 2 * r * c * 3 + 2 * c,
        tolerances=((1.0e-2, 1.0e-2),),
        seed=1234,
        modeled_bytes_per_element=12.0,
        reread_bytes_per_element=6.0,
        staged_bytes_per_element=2,
        reductions_per_stage=(2, 2),
        staged_max_cols=32768,
        stream_mix=(2, 1),
        split_pipeline_depth=_layernorm_bwd_bf16_depth,
    ),
    "softmax_logits_backward": WorkloadSpec(
        name="softmax_logits_backward",
        label="Softmax-logits backward",
        category="softmax",
        rows=4096,
        cols=65536,
        input_factory=make_softmax_logits_inputs,
        output_names=("dx",),
        algorithmic_bytes=lambda r, c: 4 * r * c * 3,
        tolerances=((3.0e-3, 3.0e-3),),
        seed=1234,
        modeled_bytes_per_element=24.0,
        reread_bytes_per_element=12.0,
        staged_bytes_per_element=8,
        reductions_per_stage=(2, 1),
        staged_max_cols=32768,
        stream_mix=(2, 1),
    ),
    # dsmem_eval/workloads.py:150-154,203-211; metadata
    # dsmem_eval/workload_metadata.py:32-34.  q is bit-exact; the scale is
    # one fp32 division (max_abs / 127).
    "rowwise_quant": WorkloadSpec(
        name="rowwise_quant",
        label="Row-wise int8 quantization",
        category="quantization",
        rows=4096,
        cols=65536,
        input_factory=make_quant_inputs,
        output_names=("q", "scale"),
        algorithmic_bytes=lambda r, c: 4 * r * c + r * c + 4 * r,
        tolerances=(None, (1.0e-6, 1.0e-6)),
        seed=1234,
        modeled_bytes_per_element=9.0,
        reread_bytes_per_element=4.0,
        staged_bytes_per_element=4,
        reductions_per_stage=(1,),
        staged_max_cols=65536,
        stream_mix=(4, 1),
    ),
    # dsmem_eval/workloads.py:128-143,194-202.  This build's READ variant
    # streams w, g, m twice (24 B) and writes w', u (8 B); staging w and u
    # saves the 12-byte re-read.
    "lars_momentum": WorkloadSpec(
        name="lars_momentum",
        label="LARS momentum",
        category="optimizer",
        rows=4096,
        cols=65536,
        input_factory=make_lars_inputs,
        output_names=("weight_out", "update"),
        algorithmic_bytes=lambda r, c: 4 * r * c * 5,
        tolerances=(FP32_TOL, FP32_TOL),
        seed=1234,
        modeled_bytes_per_element=32.0,
        reread_bytes_per_element=12.0,
        staged_bytes_per_element=8,
        reductions_per_stage=(2,),
        staged_max_cols=32768,
        stream_mix=(3, 2),
    ),
    # dsmem_eval/workloads.py:64-85,167-175.  One exchange of five sums per
    # row (the reference: three stages, (2, 1, 2)).
    "weighted_var_backward": WorkloadSpec(
        name="weighted_var_backward",
        label="Weighted variance backward",
        category="normalization",
        rows=4096,
        cols=65536,
        input_factory=make_weighted_var_inputs,
        output_names=("dx",),
        algorithmic_bytes=lambda r, c: 4 * r * c * 4,
        tolerances=(FP32_TOL,),
        seed=1234,
        modeled_bytes_per_element=28.0,
        reread_bytes_per_element=12.0,
        staged_bytes_per_element=12,
        reductions_per_stage=(5,),
        staged_max_cols=16384,
        stream_mix=(3, 1),
    ),
    # dsmem_eval/workloads.py:88-112,176-184.  One exchange of five sums per
    # row (the reference: two stages, (2, 3)).
    "pearson_backward": WorkloadSpec(
        name="pearson_backward",
        label="Pearson backward",
        category="pairwise statistics",
        rows=4096,
        cols=65536,
        input_factory=make_pearson_inputs,
        output_names=("dx", "dy"),
        algorithmic_bytes=lambda r, c: 4 * r * c * 4 + 4 * r,
        tolerances=(FP32_TOL, FP32_TOL),
        seed=1234,
        modeled_bytes_per_element=24.0,
        reread_bytes_per_element=8.0,
        staged_bytes_per_element=8,
        reductions_per_stage=(5,),
        staged_max_cols=32768,
        stream_mix=(2, 2),
    ),
}

# FFN flop count of one call: two GEMMs, 2*M*d*f each.
FFN_DIM = 28672


def ffn_flops(rows: int, d: int, f: int = FFN_DIM) -> int:
    return 2 * rows * d * f * 2


def ffn_backward_flops(rows: int, d: int, f: int = FFN_DIM) -> int:
    """The four gradient GEMMs (dh, da, dW1, dW2), 2*M*d*f each; the
    recompute of the forward's first GEMM is extra work, not counted."""
    return 2 * rows * d * f * 4

