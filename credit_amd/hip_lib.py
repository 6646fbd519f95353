"""ctypes binding of libcredit_hip.so, the gfx950 wide-row kernels.

This is the in-process operator boundary.  It mirrors the reference's
Triton launcher table (dsmem_eval/triton_kernels.py:300-414):
``HIP_LAUNCHERS[name](inputs, outputs, ...)`` writes the outputs in place and
``allocate_outputs(name, inputs)`` gives their shapes and dtypes.  The
reference's CUDA kernels sat behind a subprocess + stdout protocol
(dsmem_eval/runner.py:280-310); here they are direct calls on the caller's
current HIP stream.

The library is loaded from the package directory (built by
``credit_amd/csrc/Makefile``).  There is no fallback: a missing library or a
non-zero status raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import torch

LIB_PATH = Path(__file__).resolve().parent / "libcredit_hip.so"

# Status codes (include/credit.h).
CREDIT_OK = 0
STATUS_NAMES = {
    0: "CREDIT_OK",
    -1: "CREDIT_ERR_NULL_POINTER",
    -2: "CREDIT_ERR_BAD_SHAPE",
    -3: "CREDIT_ERR_ALIGNMENT",
    -4: "CREDIT_ERR_UNSUPPORTED",
    -5: "CREDIT_ERR_WORKSPACE",
    -6: "CREDIT_ERR_HIP",
    -7: "CREDIT_ERR_WATCHDOG",
    -8: "CREDIT_ERR_BAD_CONFIG",
}

VARIANTS = {"auto": 0, "read": 1, "staged": 2, "split": 3}
VARIANT_NAMES = {v: k for k, v in VARIANTS.items()}

OPS = {
    "row_sum_max": 1,
    "layernorm_fwd": 2,
    "layernorm_backward": 3,
    "rmsnorm_fwd": 4,
    "rmsnorm_bwd": 5,
    "softmax_fwd": 6,
    "softmax_bwd": 7,
    "softmax_logits_backward": 8,
    "ffn": 9,
    "layernorm_backward_bf16": 10,
    "rowwise_quant": 11,
    "lars_momentum": 12,
    "weighted_var_backward": 13,
    "pearson_backward": 14,
    "rmsnorm_fwd_bwd": 15,
}


class CreditError(RuntimeError):
    """A non-zero status from libcredit_hip.so."""

    def __init__(self, status: int, function: str, message: str):
        self.status = status
        self.function = function
        super().__init__(f"{function}: {STATUS_NAMES.get(status, status)}: {message}")


class CreditCfg(ctypes.Structure):
    _fields_ = [
        ("stream", ctypes.c_void_p),
        ("variant", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 128),
        ("arch", ctypes.c_char * 64),
        ("device", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("xcd_count", ctypes.c_int32),
        ("wave_size", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("cooperative_launch", ctypes.c_int32),
        ("lds_bytes_per_block", ctypes.c_int64),
        ("lds_bytes_per_cu", ctypes.c_int64),
        ("l2_bytes", ctypes.c_int64),
        ("hbm_bytes", ctypes.c_int64),
        ("clock_khz", ctypes.c_int32),
        ("mem_clock_khz", ctypes.c_int32),
        ("mem_bus_width_bits", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_CFG = ctypes.POINTER(CreditCfg)

# name -> argument types (return type is int unless listed in _RESTYPES).
SIGNATURES: dict[str, list] = {
    "credit_version": [],
    "credit_last_error": [],
    "credit_status_string": [ctypes.c_int],
    "credit_query_device": [ctypes.c_int32, ctypes.POINTER(DeviceInfo)],
    "credit_workspace_bytes": [ctypes.c_int32, _I64, _I64, ctypes.c_int32, ctypes.c_int32],
    "credit_check_watchdog": [_CFG],
    "credit_set_spin_limit": [ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)],
    "credit_row_sum_max_f32": [_P, _P, _P, _I64, _I64, _CFG],
    "credit_layernorm_fwd_bf16": [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_rmsnorm_fwd_bf16": [_P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_rmsnorm_bwd_bf16": [_P, _P, _P, _P, _P, _P, _I64, _I64, _CFG],
    "credit_rmsnorm_bwd_bf16_noalloc": [_P, _P, _P, _P, _P, _P, _I64, _I64, _CFG],
    "credit_rmsnorm_fwd_bwd_bf16": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_softmax_fwd_f32": [_P, _P, _P, _P, _I64, _I64, _CFG],
    "credit_softmax_bwd_f32": [_P, _P, _P, _I64, _I64, _CFG],
    "credit_softmax_logits_bwd_f32": [_P, _P, _P, _I64, _I64, _CFG],
    "credit_rowwise_quant_f32": [_P, _P, _P, _I64, _I64, _CFG],
    "credit_lars_momentum_f32": [_P, _P, _P, _P, _P, _I64, _I64, _CFG],
    "credit_weighted_var_bwd_f32": [_P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_pearson_bwd_f32": [_P, _P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_ffn_rmsnorm_gelu_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _F, _CFG],
    "credit_ffn_rmsnorm_gelu_kn_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _F, _CFG],
    "credit_ffn_rmsnorm_gelu_bwd_bf16": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _CFG],
    "credit_ffn_rmsnorm_gelu_fwd_train_bf16": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F,
                                               _CFG],
    "credit_ffn_rmsnorm_gelu_bwd_saved_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                               _I64, _CFG],
    "credit_ffn_rmsnorm_gelu_fwd_train_kn_bf16": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                                  _F, _CFG],
    "credit_ffn_rmsnorm_gelu_bwd_kn_bf16": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F,
                                            _CFG],
    "credit_ffn_rmsnorm_gelu_bwd_saved_kn_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                                  _I64, _I64, _CFG],
    "credit_ffn_bwd_workspace_bytes": [_I64, _I64, _I64],
    "credit_layernorm_bwd_f32": [_P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_layernorm_bwd_bf16": [_P, _P, _P, _P, _I64, _I64, _F, _CFG],
    "credit_transpose_bf16": [_P, _P, _I64, _I64, _CFG],
    "credit_microbench": [ctypes.c_int32, _I64, ctypes.c_int32, ctypes.POINTER(ctypes.c_double),
                          ctypes.c_int32],
    "credit_stream_ceiling": [ctypes.c_int32, ctypes.c_int32, _I64, ctypes.c_int32, ctypes.c_int32,
                              ctypes.c_double, ctypes.POINTER(ctypes.c_double), ctypes.c_int32],
    "credit_control_overhead": [_I64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
    "credit_last_split_shape": [ctypes.POINTER(ctypes.c_int32)] * 4,
    "credit_set_clock_probe": [_P],
    "credit_host_watchdog_words": [ctypes.POINTER(ctypes.c_int32)],
}
_RESTYPES = {
    "credit_version": ctypes.c_char_p,
    "credit_last_error": ctypes.c_char_p,
    "credit_status_string": ctypes.c_char_p,
    "credit_workspace_bytes": ctypes.c_size_t,
    "credit_ffn_bwd_workspace_bytes": ctypes.c_size_t,
}

_lib: ctypes.CDLL | None = None
# Per-thread stand-in for the library while bind() records a launcher.
_recording = threading.local()


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libcredit_hip.so once and declare every entry point's signature.

    torch is imported first so that the HIP runtime torch already mapped is
    the one the library binds to (both carry the soname libamdhip64.so.7).
    """
    global _lib
    if path is None:
        recorder = getattr(_recording, "recorder", None)
        if recorder is not None:
            return recorder
        if _lib is not None:
            return _lib
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.is_file():
        raise FileNotFoundError(
            f"{lib_path} is missing; build it with `make -C credit_amd/csrc` "
            "or `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    lib = ctypes.CDLL(str(lib_path), mode=ctypes.RTLD_GLOBAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    return load_library().credit_last_error().decode()


def check(status: int, function: str) -> None:
    if status != CREDIT_OK:
        raise CreditError(status, function, last_error())


def query_device(device: int = 0) -> dict:
    info = DeviceInfo()
    check(load_library().credit_query_device(device, ctypes.byref(info)), "credit_query_device")
    out = {name: getattr(info, name) for name, _ in DeviceInfo._fields_ if name != "reserved"}
    out["name"] = info.name.decode()
    out["arch"] = info.arch.decode()
    return out


def make_cfg(
    variant: str | int = "auto",
    split: int = 0,
    stream: int | None = None,
    workspace: torch.Tensor | None = None,
) -> CreditCfg:
    """Build a credit_cfg for the current torch stream (or `stream`)."""
    if isinstance(variant, str):
        if variant not in VARIANTS:
            raise ValueError(f"unknown variant {variant!r}; expected one of {sorted(VARIANTS)}")
        variant = VARIANTS[variant]
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else 0
    cfg = CreditCfg()
    cfg.stream = stream or None
    cfg.variant = int(variant)
    cfg.split = int(split)
    if workspace is not None:
        cfg.workspace = workspace.data_ptr()
        cfg.workspace_bytes = workspace.numel() * workspace.element_size()
    return cfg


def workspace_bytes(op: str, rows: int, cols: int, variant: str = "auto", split: int = 0) -> int:
    return int(load_library().credit_workspace_bytes(OPS[op], rows, cols, VARIANTS[variant], split))


def check_watchdog(cfg: CreditCfg | None = None) -> None:
    cfg = cfg if cfg is not None else make_cfg()
    check(load_library().credit_check_watchdog(ctypes.byref(cfg)), "credit_check_watchdog")


def set_spin_limit(polls: int) -> int:
    """Polls a split launch's bounded wait makes before giving up, for
    launches enqueued from now on (credit_set_spin_limit); returns the old
    value.  0 forces the failure path: wrong outputs and CREDIT_ERR_WATCHDOG."""
    prev = ctypes.c_uint32(0)
    check(load_library().credit_set_spin_limit(int(polls), ctypes.byref(prev)),
          "credit_set_spin_limit")
    return prev.value


def _ptr(t: torch.Tensor, name: str, dtype: torch.dtype) -> int:
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: tensor must be on a GPU, got {t.device}")
    return t.data_ptr()


def _rows_cols(x: torch.Tensor) -> tuple[int, int]:
    if x.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(x.shape)}")
    return int(x.shape[0]), int(x.shape[1])


MICROBENCH = {
    "hbm_read": 1,
    "hbm_write": 2,
    "hbm_copy": 3,
    "clock": 4,
    "latency": 5,
    "lds_read": 6,
    "lds_write": 7,
    "exchange_roundtrip": 8,
    "cache_read": 9,
    "exchange_throughput": 10,
    "mfma_bf16": 11,
    "xcc_map": 12,
    "runtime_copy": 13,
}


def microbench(name: str, nbytes: int = 0, iters: int = 0, n_results: int = 16) -> list[float]:
    """Run one gfx950 calibration microbenchmark (include/credit.h)."""
    out = (ctypes.c_double * n_results)()
    check(load_library().credit_microbench(MICROBENCH[name], nbytes, iters, out, n_results),
          "credit_microbench")
    return list(out)


def mfma_ceiling(iters: int = 20000) -> dict:
    """Attainable dense bf16 MFMA rate (CREDIT_MB_MFMA_BF16): TFLOP/s of
    back-to-back v_mfma_f32_32x32x16_bf16 chains on every CU, the shader
    clock the waves ran at, and the waves per SIMD that reached it."""
    r = microbench("mfma_bf16", 0, iters, 6)
    return {"TFLOPs": round(r[0], 1), "clock_MHz": round(r[1], 1),
            "flops_per_cycle_cu": round(r[2], 1), "waves_per_simd": int(r[3]),
            "TFLOPs_by_waves_per_simd": {"1": round(r[4], 1), "2": round(r[5], 1)}}


def stream_ceiling(reads: int, writes: int, call_bytes: int, trials: int = 5, iters: int = 20,
                   settle_ms: float = 20.0) -> dict:
    """Settled HBM stream ceiling of a reads:writes byte mix at call_bytes
    per call (credit_stream_ceiling): the best GB/s over the library's
    stream-kernel shapes and the shape that reached it."""
    out = (ctypes.c_double * 32)()
    check(load_library().credit_stream_ceiling(reads, writes, int(call_bytes), trials, iters,
                                               float(settle_ms), out, 32),
          "credit_stream_ceiling")
    return {"mix": f"{reads}:{writes}", "GBps": round(out[0], 1), "ms": out[1],
            "shape": {"lanes": int(out[2]), "vectors_per_lane": int(out[3]),
                      "workgroups_per_cu": int(out[4]), "nontemporal_stores": bool(out[5])},
            "bytes": int(out[6])}


def control_overhead(rows: int, split: int, barriers: int, warmup: int = 3, iters: int = 20,
                     cooperative: bool = False, lds_bytes: int = 0,
                     threads: int = 0) -> tuple[float, float]:
    """(plain_ms, split_ms): `rows` rows covered by a co-resident wave of
    ticketed groups of `split` workgroups meeting `barriers` times per row,
    against a plain launch of rows * split workgroups with no exchange
    (replaces build/cluster_control).  The barrier workgroups have `threads`
    lanes (0: 256) and `lds_bytes` of dynamic LDS, the reference's
    --shared-bytes (src/cluster_control.cu:76-88)."""
    plain = ctypes.c_double()
    split_ms = ctypes.c_double()
    check(load_library().credit_control_overhead(rows, split, barriers, int(lds_bytes),
                                                 int(threads), warmup, iters, int(cooperative),
                                                 ctypes.byref(plain), ctypes.byref(split_ms)),
          "credit_control_overhead")
    return plain.value, split_ms.value


def last_split_shape() -> dict:
    """Shape of this thread's last co-resident split launch
    (credit_last_split_shape): block size, LDS per workgroup, workgroups per
    CU and ticket subsets."""
    vals = [ctypes.c_int32() for _ in range(4)]
    check(load_library().credit_last_split_shape(*[ctypes.byref(v) for v in vals]),
          "credit_last_split_shape")
    return dict(zip(("threads", "lds_bytes", "per_cu", "dispensers"), (v.value for v in vals)))


def gemm_clock_mhz(run, device=None) -> float:
    """Mean shader clock (MHz) the FFN's 256-tile GEMM workgroups ran at
    during run() (credit_set_clock_probe: each workgroup's s_memtime cycles
    over its 100 MHz s_memrealtime ticks, start to end, summed)."""
    sums = torch.zeros(2, dtype=torch.int64, device=device or "cuda")
    torch.cuda.synchronize()
    check(load_library().credit_set_clock_probe(sums.data_ptr()), "credit_set_clock_probe")
    try:
        run()
        torch.cuda.synchronize()
    finally:
        check(load_library().credit_set_clock_probe(None), "credit_set_clock_probe")
    cycles, ticks = (int(v) & 0xFFFFFFFFFFFFFFFF for v in sums.cpu().tolist())
    return 100.0 * cycles / ticks if ticks else float("nan")


def control_lds_bytes(shape: dict, lds_per_cu: int) -> int:
    """Dynamic LDS for credit_control_overhead that gives the barrier grid
    the split launch's residency: the launch's own LDS, raised (when the
    launch's occupancy is set by registers rather than LDS) into the window
    (lds_per_cu / (per_cu + 1), lds_per_cu / per_cu] that admits exactly
    per_cu workgroups per CU.  1 KiB of margin on both sides covers the
    barrier kernel's static LDS and the allocation granularity."""
    per_cu = max(int(shape["per_cu"]), 1)
    lds = int(shape["lds_bytes"])
    lo = lds_per_cu // (per_cu + 1) + 1024
    hi = lds_per_cu // per_cu - 1024
    if lo <= hi:
        lds = min(max(lds, lo), hi)
    return max(lds, 0)


# --------------------------------------------------------------- operators --


def row_sum_max(x: torch.Tensor, out_sum: torch.Tensor, out_max: torch.Tensor, cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_row_sum_max_f32(
            _ptr(x, "x", torch.float32),
            _ptr(out_sum, "sum", torch.float32),
            _ptr(out_max, "max", torch.float32),
            rows,
            cols,
            ctypes.byref(cfg),
        ),
        "credit_row_sum_max_f32",
    )


def layernorm_fwd(
    x: torch.Tensor,
    gamma: torch.Tensor,
    beta: torch.Tensor,
    y: torch.Tensor,
    mean: torch.Tensor,
    rstd: torch.Tensor,
    eps: float,
    cfg: CreditCfg,
) -> None:
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_layernorm_fwd_bf16(
            _ptr(x, "x", torch.bfloat16),
            _ptr(gamma, "gamma", torch.bfloat16),
            _ptr(beta, "beta", torch.bfloat16),
            _ptr(y, "y", torch.bfloat16),
            _ptr(mean, "mean", torch.float32),
            _ptr(rstd, "rstd", torch.float32),
            rows,
            cols,
            float(eps),
            ctypes.byref(cfg),
        ),
        "credit_layernorm_fwd_bf16",
    )


def rmsnorm_fwd(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor, rstd: torch.Tensor,
                eps: float, cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_rmsnorm_fwd_bf16(
            _ptr(x, "x", torch.bfloat16), _ptr(w, "w", torch.bfloat16),
            _ptr(y, "y", torch.bfloat16), _ptr(rstd, "rstd", torch.float32),
            rows, cols, float(eps), ctypes.byref(cfg)),
        "credit_rmsnorm_fwd_bf16",
    )


def rmsnorm_bwd(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, rstd: torch.Tensor,
                dx: torch.Tensor, dw: torch.Tensor, cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_rmsnorm_bwd_bf16(
            _ptr(x, "x", torch.bfloat16), _ptr(w, "w", torch.bfloat16),
            _ptr(dy, "dy", torch.bfloat16), _ptr(rstd, "rstd", torch.float32),
            _ptr(dx, "dx", torch.bfloat16), _ptr(dw, "dw", torch.float32),
            rows, cols, ctypes.byref(cfg)),
        "credit_rmsnorm_bwd_bf16",
    )


def rmsnorm_fwd_bwd(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, y: torch.Tensor,
                    rstd: torch.Tensor, dx: torch.Tensor, dw: torch.Tensor, eps: float,
                    cfg: CreditCfg) -> None:
    """Forward and backward of RMSNorm in one call: y, rstd, dx, dw."""
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_rmsnorm_fwd_bwd_bf16(
            _ptr(x, "x", torch.bfloat16), _ptr(w, "w", torch.bfloat16),
            _ptr(dy, "dy", torch.bfloat16), _ptr(y, "y", torch.bfloat16),
            _ptr(rstd, "rstd", torch.float32), _ptr(dx, "dx", torch.bfloat16),
            _ptr(dw, "dw", torch.float32), rows, cols, float(eps), ctypes.byref(cfg)),
        "credit_rmsnorm_fwd_bwd_bf16",
    )


def softmax_fwd(x: torch.Tensor, p: torch.Tensor, rowmax: torch.Tensor, lse: torch.Tensor,
                cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(x)
    check(
        load_library().credit_softmax_fwd_f32(
            _ptr(x, "x", torch.float32), _ptr(p, "p", torch.float32),
            _ptr(rowmax, "rowmax", torch.float32), _ptr(lse, "lse", torch.float32),
            rows, cols, ctypes.byref(cfg)),
        "credit_softmax_fwd_f32",
    )


def softmax_bwd(p: torch.Tensor, dy: torch.Tensor, dx: torch.Tensor, cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(p)
    check(
        load_library().credit_softmax_bwd_f32(
            _ptr(p, "p", torch.float32), _ptr(dy, "dy", torch.float32),
            _ptr(dx, "dx", torch.float32), rows, cols, ctypes.byref(cfg)),
        "credit_softmax_bwd_f32",
    )


def softmax_logits_backward(logits: torch.Tensor, dy: torch.Tensor, dx: torch.Tensor,
                            cfg: CreditCfg) -> None:
    rows, cols = _rows_cols(logits)
    check(
        load_library().credit_softmax_logits_bwd_f32(
            _ptr(logits, "logits", torch.float32), _ptr(dy, "dy", torch.float32),
            _ptr(dx, "dx", torch.float32), rows, cols, ctypes.byref(cfg)),
        "credit_softmax_logits_bwd_f32",
    )


def rowwise_quant(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor,
                  cfg: CreditCfg) -> None:
    """fp32 rows in, int8 codes and one fp32 scale per row out."""
    rows, cols = _rows_cols(x)
    if tuple(q.shape) != (rows, cols):
        raise ValueError(f"q: expected shape {(rows, cols)}, got {tuple(q.shape)}")
    if scale.numel() != rows:
        raise ValueError(f"scale: expected {rows} elements, got {scale.numel()}")
    check(
        load_library().credit_rowwise_quant_f32(
            _ptr(x, "x", torch.float32), _ptr(q, "q", torch.int8),
            _ptr(scale, "scale", torch.float32), rows, cols, ctypes.byref(cfg)),
        "credit_rowwise_quant_f32",
    )


def _same_shape(name: str, t: torch.Tensor, shape: tuple[int, int]) -> None:
    if tuple(t.shape) != shape:
        raise ValueError(f"{name}: expected shape {shape}, got {tuple(t.shape)}")


def lars_momentum(weight: torch.Tensor, grad: torch.Tensor, momentum: torch.Tensor,
                  weight_out: torch.Tensor, update_out: torch.Tensor, cfg: CreditCfg) -> None:
    """fp32 [rows, cols] in and out."""
    rows, cols = _rows_cols(weight)
    for name, t in (("grad", grad), ("momentum", momentum), ("weight_out", weight_out),
                    ("update_out", update_out)):
        _same_shape(name, t, (rows, cols))
    f32 = torch.float32
    check(
        load_library().credit_lars_momentum_f32(
            _ptr(weight, "weight", f32), _ptr(grad, "grad", f32), _ptr(momentum, "momentum", f32),
            _ptr(weight_out, "weight_out", f32), _ptr(update_out, "update_out", f32), rows, cols,
            ctypes.byref(cfg)),
        "credit_lars_momentum_f32",
    )


def weighted_var_backward(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor,
                          dx: torch.Tensor, eps: float, cfg: CreditCfg) -> None:
    """fp32 [rows, cols] in and out."""
    rows, cols = _rows_cols(x)
    for name, t in (("weight", weight), ("dy", dy), ("dx", dx)):
        _same_shape(name, t, (rows, cols))
    f32 = torch.float32
    check(
        load_library().credit_weighted_var_bwd_f32(
            _ptr(x, "x", f32), _ptr(weight, "weight", f32), _ptr(dy, "dy", f32),
            _ptr(dx, "dx", f32), rows, cols, eps, ctypes.byref(cfg)),
        "credit_weighted_var_bwd_f32",
    )


def pearson_backward(x: torch.Tensor, y: torch.Tensor, grad: torch.Tensor, dx: torch.Tensor,
                     dy: torch.Tensor, eps: float, cfg: CreditCfg) -> None:
    """x, y, dx, dy fp32 [rows, cols]; grad fp32 with one value per row."""
    rows, cols = _rows_cols(x)
    for name, t in (("y", y), ("dx", dx), ("dy", dy)):
        _same_shape(name, t, (rows, cols))
    if grad.numel() != rows:
        raise ValueError(f"grad: expected {rows} elements, got {grad.numel()}")
    f32 = torch.float32
    check(
        load_library().credit_pearson_bwd_f32(
            _ptr(x, "x", f32), _ptr(y, "y", f32), _ptr(grad, "grad", f32), _ptr(dx, "dx", f32),
            _ptr(dy, "dy", f32), rows, cols, eps, ctypes.byref(cfg)),
        "credit_pearson_bwd_f32",
    )


def layernorm_backward(x: torch.Tensor, dy: torch.Tensor, gamma: torch.Tensor,
                       dx: torch.Tensor, eps: float, cfg: CreditCfg) -> None:
    """fp32 or bf16 (all four tensors the same dtype)."""
    rows, cols = _rows_cols(x)
    if x.dtype == torch.float32:
        fn, name, dt = load_library().credit_layernorm_bwd_f32, "credit_layernorm_bwd_f32", x.dtype
    elif x.dtype == torch.bfloat16:
        fn, name, dt = (load_library().credit_layernorm_bwd_bf16, "credit_layernorm_bwd_bf16",
                        x.dtype)
    else:
        raise TypeError(f"layernorm_backward: unsupported dtype {x.dtype}")
    check(fn(_ptr(x, "x", dt), _ptr(dy, "dy", dt), _ptr(gamma, "gamma", dt), _ptr(dx, "dx", dt),
             rows, cols, float(eps), ctypes.byref(cfg)), name)


def ffn(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, out: torch.Tensor, eps: float,
        cfg: CreditCfg, layout: str = "linear") -> None:
    """out = x + GELU_tanh(RMSNorm(x) W1) W2.  layout "linear": the nn.Linear
    layout, w1 [f, d] and w2 [d, f] (out = ... @ w1.T ... @ w2.T); layout
    "in_out": w1 [d, f] and w2 [f, d] as the BASELINE gives them
    (credit_ffn_rmsnorm_gelu_kn_bf16, no transpose anywhere)."""
    rows, d = _rows_cols(x)
    if layout == "linear":
        f = int(w1.shape[0])
        want1, want2, fname = (f, d), (d, f), "credit_ffn_rmsnorm_gelu_bf16"
    elif layout == "in_out":
        f = int(w1.shape[1])
        want1, want2, fname = (d, f), (f, d), "credit_ffn_rmsnorm_gelu_kn_bf16"
    else:
        raise ValueError(f"ffn: layout must be 'linear' or 'in_out', got {layout!r}")
    if tuple(w1.shape) != want1 or tuple(w2.shape) != want2:
        raise ValueError(f"ffn ({layout}): w1 must be {list(want1)} and w2 {list(want2)}; got "
                         f"{tuple(w1.shape)}, {tuple(w2.shape)} for d={d}")
    check(
        getattr(load_library(), fname)(
            _ptr(x, "x", torch.bfloat16), _ptr(w1, "w1", torch.bfloat16),
            _ptr(w2, "w2", torch.bfloat16), _ptr(out, "out", torch.bfloat16),
            rows, d, f, float(eps), ctypes.byref(cfg)),
        fname,
    )


def transpose(src: torch.Tensor, dst: torch.Tensor, cfg: CreditCfg | None = None) -> None:
    rows, cols = _rows_cols(src)
    if tuple(dst.shape) != (cols, rows):
        raise ValueError("transpose: dst must be [cols, rows]")
    cfg = cfg if cfg is not None else make_cfg()
    check(
        load_library().credit_transpose_bf16(
            _ptr(src, "src", torch.bfloat16), _ptr(dst, "dst", torch.bfloat16),
            rows, cols, ctypes.byref(cfg)),
        "credit_transpose_bf16",
    )


def _ffn_dims(x, w1, w2, what, kn):
    """(rows, d, f) of an FFN call: w1 [f, d], w2 [d, f] (nn.Linear), or with
    kn w1 [d, f], w2 [f, d] ([in, out])."""
    rows, d = _rows_cols(x)
    f = int(w1.shape[1] if kn else w1.shape[0])
    want1, want2 = ((d, f), (f, d)) if kn else ((f, d), (d, f))
    if tuple(w1.shape) != want1 or tuple(w2.shape) != want2:
        raise ValueError(f"{what}: w1 must be {list(want1)} and w2 {list(want2)}; got "
                         f"{tuple(w1.shape)}, {tuple(w2.shape)}")
    return rows, d, f


def ffn_backward(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, dout: torch.Tensor,
                 dx: torch.Tensor, dw1: torch.Tensor, dw2: torch.Tensor, eps: float,
                 cfg: CreditCfg, kn: bool = False) -> None:
    """Gradients of ffn(): dx [rows, d] and dw1, dw2 in the weights' own
    layouts, all bf16.  w1 [f, d], w2 [d, f] as the forward, or with kn the
    [in, out] weights w1 [d, f], w2 [f, d]."""
    rows, d, f = _ffn_dims(x, w1, w2, "ffn_backward", kn)
    for name, t, shape in (("dout", dout, (rows, d)), ("dx", dx, (rows, d)),
                           ("dw1", dw1, tuple(w1.shape)), ("dw2", dw2, tuple(w2.shape))):
        if tuple(t.shape) != shape:
            raise ValueError(f"ffn_backward: {name} must be {shape}, got {tuple(t.shape)}")
    bf = torch.bfloat16
    fn = "credit_ffn_rmsnorm_gelu_bwd_kn_bf16" if kn else "credit_ffn_rmsnorm_gelu_bwd_bf16"
    check(
        getattr(load_library(), fn)(
            _ptr(x, "x", bf), _ptr(w1, "w1", bf), _ptr(w2, "w2", bf), _ptr(dout, "dout", bf),
            _ptr(dx, "dx", bf), _ptr(dw1, "dw1", bf), _ptr(dw2, "dw2", bf), rows, d, f,
            float(eps), ctypes.byref(cfg)),
        fn,
    )


def ffn_train_forward(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, out: torch.Tensor,
                      rstd: torch.Tensor, u: torch.Tensor, h: torch.Tensor, eps: float,
                      cfg: CreditCfg, kn: bool = False) -> None:
    """ffn() (nn.Linear weights, or with kn the [in, out] ones) that also
    writes what its backward needs: rstd [rows] fp32, u [rows, f] and h
    [rows, f] bf16."""
    rows, d, f = _ffn_dims(x, w1, w2, "ffn_train_forward", kn)
    for name, t, shape in (("out", out, (rows, d)), ("rstd", rstd, (rows,)),
                           ("u", u, (rows, f)), ("h", h, (rows, f))):
        if tuple(t.shape) != shape:
            raise ValueError(f"ffn_train_forward: {name} must be {shape}, got {tuple(t.shape)}")
    bf = torch.bfloat16
    fn = ("credit_ffn_rmsnorm_gelu_fwd_train_kn_bf16" if kn
          else "credit_ffn_rmsnorm_gelu_fwd_train_bf16")
    check(
        getattr(load_library(), fn)(
            _ptr(x, "x", bf), _ptr(w1, "w1", bf), _ptr(w2, "w2", bf), _ptr(out, "out", bf),
            _ptr(rstd, "rstd", torch.float32), _ptr(u, "u", bf), _ptr(h, "h", bf), rows, d, f,
            float(eps), ctypes.byref(cfg)),
        fn,
    )


def ffn_backward_saved(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, dout: torch.Tensor,
                       rstd: torch.Tensor, u: torch.Tensor, h: torch.Tensor, dx: torch.Tensor,
                       dw1: torch.Tensor, dw2: torch.Tensor, cfg: CreditCfg,
                       kn: bool = False) -> None:
    """ffn_backward() from the saved rstd, u and h of ffn_train_forward()
    (the same weight layout, kn)."""
    rows, d, f = _ffn_dims(x, w1, w2, "ffn_backward_saved", kn)
    for name, t, shape in (("dout", dout, (rows, d)), ("rstd", rstd, (rows,)),
                           ("u", u, (rows, f)), ("h", h, (rows, f)), ("dx", dx, (rows, d)),
                           ("dw1", dw1, tuple(w1.shape)), ("dw2", dw2, tuple(w2.shape))):
        if tuple(t.shape) != shape:
            raise ValueError(f"ffn_backward_saved: {name} must be {shape}, got {tuple(t.shape)}")
    bf = torch.bfloat16
    fn = ("credit_ffn_rmsnorm_gelu_bwd_saved_kn_bf16" if kn
          else "credit_ffn_rmsnorm_gelu_bwd_saved_bf16")
    check(
        getattr(load_library(), fn)(
            _ptr(x, "x", bf), _ptr(w1, "w1", bf), _ptr(w2, "w2", bf), _ptr(dout, "dout", bf),
            _ptr(rstd, "rstd", torch.float32), _ptr(u, "u", bf), _ptr(h, "h", bf),
            _ptr(dx, "dx", bf), _ptr(dw1, "dw1", bf), _ptr(dw2, "dw2", bf), rows, d, f,
            ctypes.byref(cfg)),
        fn,
    )


def linear_layout(w: torch.Tensor) -> torch.Tensor:
    """A [in, out] weight (the BASELINE's W1 [d, f]) in the nn.Linear layout
    [out, in] the FFN takes, transposed on the GPU by this library."""
    out = torch.empty((w.shape[1], w.shape[0]), dtype=w.dtype, device=w.device)
    transpose(w, out)
    return out


# ------------------------------------------------- reference-shaped table --


@dataclass(frozen=True)
class LaunchConfig:
    """Knobs a launcher takes: the variant and split factor replace the
    reference's (block_size, num_warps) Triton pair and cluster size P."""

    variant: str = "auto"
    split: int = 0


def launch_row_sum_max(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    (x,) = inputs
    s, m = outputs
    row_sum_max(x, s, m, make_cfg(config.variant, config.split))


def launch_layernorm_fwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x, gamma, beta = inputs
    y, mean, rstd = outputs
    layernorm_fwd(x, gamma, beta, y, mean, rstd, 1.0e-5, make_cfg(config.variant, config.split))


RMSNORM_EPS = 1.0e-6


def launch_rmsnorm_fwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x, w = inputs[0], inputs[1]
    y, rstd = outputs
    rmsnorm_fwd(x, w, y, rstd, RMSNORM_EPS, make_cfg(config.variant, config.split))


def launch_rmsnorm_bwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w, dy, rstd) -- rstd from the forward."""
    x, w, dy, rstd = inputs
    dx, dw = outputs
    rmsnorm_bwd(x, w, dy, rstd, dx, dw, make_cfg(config.variant, config.split))


def launch_rmsnorm_fwd_bwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w, dy); outputs: (y, rstd, dx, dw)."""
    x, w, dy = inputs
    y, rstd, dx, dw = outputs
    rmsnorm_fwd_bwd(x, w, dy, y, rstd, dx, dw, RMSNORM_EPS, make_cfg(config.variant, config.split))


def launch_softmax_fwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x = inputs[0]
    p, rowmax, lse = outputs
    softmax_fwd(x, p, rowmax, lse, make_cfg(config.variant, config.split))


def launch_softmax_bwd(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (p, dy) -- p from the forward."""
    p, dy = inputs[0], inputs[1]
    (dx,) = outputs
    softmax_bwd(p, dy, dx, make_cfg(config.variant, config.split))


def launch_softmax_logits_backward(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    logits, dy = inputs
    (dx,) = outputs
    softmax_logits_backward(logits, dy, dx, make_cfg(config.variant, config.split))


def launch_rowwise_quant(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    (x,) = inputs
    q, scale = outputs
    rowwise_quant(x, q, scale, make_cfg(config.variant, config.split))


def launch_lars_momentum(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    lars_momentum(*inputs, *outputs, make_cfg(config.variant, config.split))


WEIGHTED_VAR_EPS = 1.0e-5  # dsmem_eval/workloads.py:74,78
PEARSON_EPS = 1.0e-6       # dsmem_eval/workloads.py:104-105


def launch_weighted_var_backward(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x, w, dy = inputs
    (dx,) = outputs
    weighted_var_backward(x, w, dy, dx, WEIGHTED_VAR_EPS, make_cfg(config.variant, config.split))


def launch_pearson_backward(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x, y, grad = inputs
    dx, dy = outputs
    pearson_backward(x, y, grad, dx, dy, PEARSON_EPS, make_cfg(config.variant, config.split))


FFN_EPS = 1.0e-6


def launch_ffn(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w1 [f, d], w2 [d, f]) in the nn.Linear layout."""
    x, w1, w2 = inputs
    (out,) = outputs
    ffn(x, w1, w2, out, FFN_EPS, make_cfg(config.variant, config.split))


def launch_ffn_baseline_layout(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w1 [d, f], w2 [f, d]) in the BASELINE's [in, out] layout."""
    x, w1, w2 = inputs
    (out,) = outputs
    ffn(x, w1, w2, out, FFN_EPS, make_cfg(config.variant, config.split), layout="in_out")


LAYERNORM_EPS = 1.0e-5  # dsmem_eval/workloads.py:55


def launch_ffn_backward(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w1 [f, d], w2 [d, f], dout); outputs: (dx, dw1, dw2)."""
    x, w1, w2, dout = inputs
    dx, dw1, dw2 = outputs
    ffn_backward(x, w1, w2, dout, dx, dw1, dw2, FFN_EPS, make_cfg(config.variant, config.split))


def launch_ffn_backward_baseline_layout(inputs, outputs,
                                        config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w1 [d, f], w2 [f, d], dout) in the BASELINE's [in, out]
    layout; outputs: (dx, dw1 [d, f], dw2 [f, d])."""
    x, w1, w2, dout = inputs
    dx, dw1, dw2 = outputs
    ffn_backward(x, w1, w2, dout, dx, dw1, dw2, FFN_EPS, make_cfg(config.variant, config.split),
                 kn=True)


def launch_ffn_backward_saved(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    """inputs: (x, w1 [f, d], w2 [d, f], dout, rstd, u, h) -- the last three
    from ffn_train_forward; outputs: (dx, dw1, dw2)."""
    x, w1, w2, dout, rstd, u, h = inputs
    dx, dw1, dw2 = outputs
    ffn_backward_saved(x, w1, w2, dout, rstd, u, h, dx, dw1, dw2,
                       make_cfg(config.variant, config.split))


def launch_layernorm_backward(inputs, outputs, config: LaunchConfig = LaunchConfig()) -> None:
    x, dy, gamma = inputs
    (dx,) = outputs
    layernorm_backward(x, dy, gamma, dx, LAYERNORM_EPS, make_cfg(config.variant, config.split))


HIP_LAUNCHERS: dict[str, Callable[..., None]] = {
    "ffn": launch_ffn,
    "ffn_baseline_layout": launch_ffn_baseline_layout,
    "ffn_backward": launch_ffn_backward,
    "ffn_backward_baseline_layout": launch_ffn_backward_baseline_layout,
    "ffn_backward_saved": launch_ffn_backward_saved,
    "layernorm_backward": launch_layernorm_backward,
    "layernorm_backward_bf16": launch_layernorm_backward,
    "row_sum_max": launch_row_sum_max,
    "layernorm_fwd": launch_layernorm_fwd,
    "rmsnorm_fwd": launch_rmsnorm_fwd,
    "rmsnorm_bwd": launch_rmsnorm_bwd,
    "rmsnorm_fwd_bwd": launch_rmsnorm_fwd_bwd,
    "softmax_fwd": launch_softmax_fwd,
    "softmax_bwd": launch_softmax_bwd,
    "softmax_logits_backward": launch_softmax_logits_backward,
    "rowwise_quant": launch_rowwise_quant,
    "lars_momentum": launch_lars_momentum,
    "weighted_var_backward": launch_weighted_var_backward,
    "pearson_backward": launch_pearson_backward,
}


class _Recorder:
    """Stands in for the loaded library while a launcher runs under bind():
    every entry point it calls is recorded with its converted arguments and
    reports CREDIT_OK."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib
        self.calls: list[tuple[Callable[..., int], str, tuple]] = []

    def __getattr__(self, name: str):
        fn = getattr(self._lib, name)

        def record(*args):
            self.calls.append((fn, name, args))
            return CREDIT_OK

        return record


def bind(name: str, inputs: tuple[torch.Tensor, ...], outputs: tuple[torch.Tensor, ...],
         config: LaunchConfig = LaunchConfig()) -> Callable[[], None]:
    """HIP_LAUNCHERS[name](inputs, outputs, config) as a call with its
    arguments checked and converted once: the returned function makes only
    the library calls themselves (one ctypes call per entry point), on the
    torch stream that was current here.  A timing loop over a kernel shorter
    than the launcher's Python checks measures the kernel this way, not the
    checks.  The tensors must stay alive and in place while it is used.
    Recording is per thread: launchers called on other threads meanwhile
    run as usual."""
    recorder = _Recorder(load_library())
    _recording.recorder = recorder
    try:
        HIP_LAUNCHERS[name](inputs, outputs, config)
    finally:
        _recording.recorder = None
    calls = tuple(recorder.calls)
    keep = (inputs, outputs)

    def call() -> None:
        for fn, fname, args in calls:
            status = fn(*args)
            if isinstance(status, int) and status != CREDIT_OK:
                raise CreditError(status, fname, last_error())

    call.tensors = keep  # type: ignore[attr-defined]
    return call


def prepare_inputs(name: str, cpu_inputs: tuple[torch.Tensor, ...],
                   device: torch.device | str) -> tuple[torch.Tensor, ...]:
    """The workload registry's inputs (credit_amd.workloads) as launcher
    inputs on `device`.  The backward passes take what their forward
    produced (rstd, p), computed here by this library's own forward kernels;
    the FFN weights are moved to the nn.Linear layout."""
    ins = tuple(t.to(device) for t in cpu_inputs)
    if name == "rmsnorm_fwd":
        return ins[:2]
    if name == "rmsnorm_bwd":
        x, w, dy = ins
        y, rstd = allocate_outputs("rmsnorm_fwd", (x, w))
        HIP_LAUNCHERS["rmsnorm_fwd"]((x, w), (y, rstd))
        return x, w, dy, rstd
    if name == "softmax_fwd":
        return ins[:1]
    if name == "softmax_bwd":
        x, dy = ins
        p, m, lse = allocate_outputs("softmax_fwd", (x,))
        HIP_LAUNCHERS["softmax_fwd"]((x,), (p, m, lse))
        return p, dy
    if name == "ffn":
        x, w1, w2 = ins  # W1 [d, f], W2 [f, d]
        return x, linear_layout(w1), linear_layout(w2)
    if name == "ffn_backward":
        x, w1, w2, dout = ins
        return x, linear_layout(w1), linear_layout(w2), dout
    if name == "ffn_backward_saved":
        x, w1, w2, dout = ins
        w1, w2 = linear_layout(w1), linear_layout(w2)
        rows, f = x.shape[0], w1.shape[0]
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        u = torch.empty((rows, f), device=x.device, dtype=torch.bfloat16)
        h = torch.empty_like(u)
        ffn_train_forward(x, w1, w2, torch.empty_like(x), rstd, u, h, FFN_EPS, make_cfg())
        return x, w1, w2, dout, rstd, u, h
    return ins


def allocate_outputs(name: str, inputs: tuple[torch.Tensor, ...]) -> tuple[torch.Tensor, ...]:
    """Output buffers of a launcher, as dsmem_eval/triton_kernels.py:403-414."""
    x = inputs[0]
    rows = x.shape[0]
    f32 = dict(device=x.device, dtype=torch.float32)
    if name == "row_sum_max":
        return torch.empty(rows, **f32), torch.empty(rows, **f32)
    if name == "layernorm_fwd":
        return torch.empty_like(x), torch.empty(rows, **f32), torch.empty(rows, **f32)
    if name == "rmsnorm_fwd":
        return torch.empty_like(x), torch.empty(rows, **f32)
    if name == "rmsnorm_bwd":
        return torch.empty_like(x), torch.empty(x.shape[1], **f32)
    if name == "rmsnorm_fwd_bwd":
        return (torch.empty_like(x), torch.empty(rows, **f32), torch.empty_like(x),
                torch.empty(x.shape[1], **f32))
    if name == "softmax_fwd":
        return torch.empty_like(x), torch.empty(rows, **f32), torch.empty(rows, **f32)
    if name == "rowwise_quant":
        return torch.empty(x.shape, device=x.device, dtype=torch.int8), torch.empty(rows, **f32)
    if name in ("ffn_backward", "ffn_backward_saved", "ffn_backward_baseline_layout"):
        w1 = inputs[1]
        return torch.empty_like(x), torch.empty_like(w1), torch.empty_like(inputs[2])
    if name in ("lars_momentum", "pearson_backward"):
        return torch.empty_like(x), torch.empty_like(x)
    if name == "weighted_var_backward":
        return (torch.empty_like(x),)
    if name in ("softmax_bwd", "softmax_logits_backward", "ffn", "ffn_baseline_layout",
                "layernorm_backward", "layernorm_backward_bf16"):
        return (torch.empty_like(x),)
    raise KeyError(name)
