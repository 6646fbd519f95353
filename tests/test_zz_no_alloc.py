"""credit_rmsnorm_bwd_bf16_noalloc through the C ABI: the allocation-free
variant of the RMSNorm backward (its workspace in the library's fixed
device array) must give the allocating entry point's outputs, bit for bit
(same kernels, deterministic dweight order), on two calls in a row, the
second with a smaller input; shapes beyond the array are rejected."""
import ctypes
import os
import subprocess
import sys
from pathlib import Path

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
        # In this suite's process earlier split calls have made the device's
        # host-mapped watchdog word, which the allocation-free call then uses;
        # test_noalloc_first_call_in_a_fresh_process covers the call without one.
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


_FRESH = r"""
import ctypes, sys, torch
from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
lib = hip_lib.load_library()
dev = torch.device("cuda:0")
x, w, dy = (t.to(dev) for t in WORKLOADS["rmsnorm_bwd"].make_inputs(64, 65536, seed=3))
rstd = torch.rand(64, device=dev) + 0.5
def run(fn):
    dx, dw = torch.full_like(x, 7.0), torch.full((65536,), float("nan"), device=dev)
    cfg = hip_lib.make_cfg("split", 8)
    hip_lib.check(fn(x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                     dw.data_ptr(), 64, 65536, ctypes.byref(cfg)), "rmsnorm_bwd")
    torch.cuda.synchronize()
    return dx.cpu(), dw.cpu()
def words():
    n = ctypes.c_int32()
    hip_lib.check(lib.credit_host_watchdog_words(ctypes.byref(n)), "words")
    return n.value
assert words() == 0
got = run(lib.credit_rmsnorm_bwd_bf16_noalloc)  # the first library call of the process
assert words() == 0, "the allocation-free call allocated a host watchdog word"
hip_lib.check_watchdog()
ref = run(lib.credit_rmsnorm_bwd_bf16)
assert words() == 1
assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
print("fresh-process allocation-free call: ok", flush=True)
"""


def test_noalloc_first_call_in_a_fresh_process(gpu):
    """In a child process whose first library call is the allocation-free
    one (split 8, so it runs the exchange): no host-mapped watchdog word
    exists yet and none is made; its outputs match the allocating entry
    point's, which then makes the word."""
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, PYTHONPATH=str(root) + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("allocation-free call in a child process", flush=True)
    out = subprocess.run([sys.executable, "-c", _FRESH], capture_output=True, text=True,
                         timeout=240, env=env, cwd=str(root))
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-4000:]
    assert "fresh-process allocation-free call: ok" in out.stdout
