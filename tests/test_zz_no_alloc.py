"""credit_rmsnorm_bwd_bf16_noalloc through the C ABI: the allocation-free
variant of the RMSNorm backward (its workspace in the library's fixed
device array) must give the allocating entry point's outputs, bit for bit
(same kernels, deterministic dweight order), on two calls in a row, the
second with a smaller input; shapes beyond the array are rejected."""
import ctypes

import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu


def _args(x, w, dy, rstd, dx, dw, cfg):
    rows, cols = x.shape
    return (x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
            dw.data_ptr(), rows, cols, ctypes.byref(cfg))


def _inputs(rows, cols, seed, gpu):
    x, w, dy = (t.to(gpu) for t in WORKLOADS["rmsnorm_bwd"].make_inputs(rows, cols, seed=seed))
    y, rstd = hip_lib.allocate_outputs("rmsnorm_fwd", (x, w))
    hip_lib.rmsnorm_fwd(x, w, y, rstd, hip_lib.RMSNORM_EPS, hip_lib.make_cfg())
    return x, w, dy, rstd


def _run(fn, x, w, dy, rstd, variant="auto", split=0):
    dx, dw = hip_lib.allocate_outputs("rmsnorm_bwd", (x, w, dy, rstd))
    dx.fill_(7.0)
    dw.fill_(float("nan"))
    status = fn(*_args(x, w, dy, rstd, dx, dw, hip_lib.make_cfg(variant, split)))
    hip_lib.check(status, fn.__name__)
    torch.cuda.synchronize()
    return dx.cpu(), dw.cpu()


@pytest.mark.parametrize("first,second", [((1024, 131072), (96, 65536)),
                                          ((256, 16384), (40, 8192))])
def test_noalloc_matches_the_allocating_entry_point(gpu, first, second):
    lib = hip_lib.load_library()
    for shape, seed in ((first, 11), (second, 12)):
        print(f"rmsnorm_bwd noalloc shape={shape}", flush=True)
        ins = _inputs(*shape, seed, gpu)
        # The allocation-free call first: in a fresh process no allocating
        # split call has run yet, so it runs without a host-mapped watchdog word.
        got = _run(lib.credit_rmsnorm_bwd_bf16_noalloc, *ins)
        ref = _run(lib.credit_rmsnorm_bwd_bf16, *ins)
        assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
    hip_lib.check_watchdog()


def test_noalloc_split_and_rejections(gpu):
    lib = hip_lib.load_library()
    ins = _inputs(64, 65536, 5, gpu)
    ref = _run(lib.credit_rmsnorm_bwd_bf16, *ins, "split", 8)
    got = _run(lib.credit_rmsnorm_bwd_bf16_noalloc, *ins, "split", 8)
    assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
    # More rows per group than the fixed array holds partials for.
    big = [torch.empty((100000, 8192), dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    rstd = torch.empty(100000, dtype=torch.float32, device=gpu)
    w = torch.ones(8192, dtype=torch.bfloat16, device=gpu)
    dx = torch.empty_like(big[0])
    dw = torch.empty(8192, dtype=torch.float32, device=gpu)
    cfg = hip_lib.make_cfg("read")
    status = lib.credit_rmsnorm_bwd_bf16_noalloc(big[0].data_ptr(), w.data_ptr(),
                                                 big[1].data_ptr(), rstd.data_ptr(),
                                                 dx.data_ptr(), dw.data_ptr(), 100000, 8192,
                                                 ctypes.byref(cfg))
    assert status == -5 and "fixed" in hip_lib.last_error()
    # A caller workspace is refused (it belongs to the allocating variant).
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=gpu)
    cfg = hip_lib.make_cfg(workspace=ws)
    x, w2, dy, r = ins
    dx2, dw2 = hip_lib.allocate_outputs("rmsnorm_bwd", ins)
    status = lib.credit_rmsnorm_bwd_bf16_noalloc(*_args(x, w2, dy, r, dx2, dw2, cfg))
    assert status == -8


def test_noalloc_expired_wait_is_reported(gpu):
    """A bounded wait forced to expire inside the allocation-free call (spin
    limit 0, from the host) raises the fixed array's watchdog word:
    credit_check_watchdog reports it and re-zeroes the array's header and
    counters, and the next call matches the allocating entry point again."""
    lib = hip_lib.load_library()
    ins = _inputs(64, 65536, 21, gpu)
    ref = _run(lib.credit_rmsnorm_bwd_bf16, *ins, "split", 8)
    hip_lib.check_watchdog()
    print("forcing an expired wait in the allocation-free call (spin limit 0)", flush=True)
    prev = hip_lib.set_spin_limit(0)
    try:
        _run(lib.credit_rmsnorm_bwd_bf16_noalloc, *ins, "split", 8)
    finally:
        hip_lib.set_spin_limit(prev)
    with pytest.raises(hip_lib.CreditError) as err:
        hip_lib.check_watchdog()
    assert err.value.status == -7  # CREDIT_ERR_WATCHDOG
    hip_lib.check_watchdog()  # cleared
    got = _run(lib.credit_rmsnorm_bwd_bf16_noalloc, *ins, "split", 8)
    assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
    hip_lib.check_watchdog()
