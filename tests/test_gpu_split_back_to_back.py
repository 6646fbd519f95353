"""Split launches queued back to back, with no host synchronisation between
them, as a training step issues them.

A split launch is one resident wave of ticketed groups that loop over their
rows; every member of a group waits for the others at each exchange, so a
member that is not running stalls its group until the exchange watchdog
expires.  Each case uses enough rows that every group takes several rows
(slot rows of the exchange ring are reused within the launch) and checks
that no launch raised the watchdog and that the last launch's result
matches the float64 oracle (fp32 rtol 1e-5 / atol 1e-6, bf16 1e-2 / 1e-2)."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS
from oracle import reference as ref

pytestmark = pytest.mark.gpu

FP32 = dict(rtol=1e-5, atol=1e-6)
BF16 = dict(rtol=1e-2, atol=1e-2)
LAUNCHES = 6


def queue(call):
    for _ in range(LAUNCHES):
        call()
    torch.cuda.synchronize()
    hip_lib.check_watchdog()


@pytest.mark.parametrize("split", [2, 4, 16])
def test_softmax_fwd_back_to_back(gpu, split):
    x = WORKLOADS["softmax_fwd"].make_inputs(2048, 16384, seed=3)[0]
    xs = x.to(gpu)
    p = torch.empty_like(xs)
    m = torch.empty(x.shape[0], device=gpu)
    lse = torch.empty(x.shape[0], device=gpu)
    cfg = hip_lib.make_cfg("split", split)
    print(f"softmax_fwd split {split}", flush=True)
    queue(lambda: hip_lib.softmax_fwd(xs, p, m, lse, cfg))
    ep, _, el = ref.softmax_fwd(x.numpy())
    np.testing.assert_allclose(p.cpu().numpy(), ep, **FP32)
    np.testing.assert_allclose(lse.cpu().numpy(), el, **FP32)


@pytest.mark.parametrize("split", [2, 8, 32])
def test_softmax_bwd_back_to_back(gpu, split):
    x, dy = WORKLOADS["softmax_bwd"].make_inputs(2048, 16384, seed=4)
    p32 = ref.softmax_fwd(x.numpy())[0].astype(np.float32)
    ps, ds = torch.from_numpy(p32).to(gpu), dy.to(gpu)
    dx = torch.empty_like(ps)
    cfg = hip_lib.make_cfg("split", split)
    print(f"softmax_bwd split {split}", flush=True)
    queue(lambda: hip_lib.softmax_bwd(ps, ds, dx, cfg))
    np.testing.assert_allclose(dx.cpu().numpy(), ref.softmax_bwd(p32, dy.numpy()), **FP32)


@pytest.mark.parametrize("split", [2, 8])
def test_softmax_logits_bwd_back_to_back(gpu, split):
    x, dy = WORKLOADS["softmax_logits_backward"].make_inputs(2048, 16384, seed=5)
    xs, ds = x.to(gpu), dy.to(gpu)
    dx = torch.empty_like(xs)
    cfg = hip_lib.make_cfg("split", split)
    print(f"softmax_logits_backward split {split}", flush=True)
    queue(lambda: hip_lib.softmax_logits_backward(xs, ds, dx, cfg))
    expect = ref.softmax_logits_backward(x.numpy(), dy.numpy())
    np.testing.assert_allclose(dx.cpu().numpy(), expect, **FP32)


@pytest.mark.parametrize("split", [2, 8])
def test_layernorm_bwd_back_to_back(gpu, split):
    x, dy, gamma = WORKLOADS["layernorm_backward"].make_inputs(2048, 16384, seed=6)
    ins = [t.to(gpu) for t in (x, dy, gamma)]
    dx = torch.empty_like(ins[0])
    cfg = hip_lib.make_cfg("split", split)
    print(f"layernorm_backward split {split}", flush=True)
    queue(lambda: hip_lib.layernorm_backward(*ins, dx, 1e-5, cfg))
    expect = ref.layernorm_backward(x.numpy(), dy.numpy(), gamma.numpy(), 1e-5)
    np.testing.assert_allclose(dx.cpu().numpy(), expect, **FP32)


def test_layernorm_bwd_bf16_group_back_to_back(gpu):
    """The bf16 group pipeline (AUTO at 65536 columns: 8 members of 1024
    vectors, rows published four steps ahead), 64 rows per group."""
    x, dy, gamma = WORKLOADS["layernorm_backward_bf16"].make_inputs(2048, 65536, seed=6)
    ins = [t.to(gpu) for t in (x, dy, gamma)]
    dx = torch.empty_like(ins[0])
    cfg = hip_lib.make_cfg()
    print("layernorm_backward_bf16 auto (2048, 65536)", flush=True)
    queue(lambda: hip_lib.layernorm_backward(*ins, dx, 1e-5, cfg))
    expect = ref.layernorm_backward(x.float().numpy(), dy.float().numpy(),
                                    gamma.float().numpy(), 1e-5)
    np.testing.assert_allclose(dx.float().cpu().numpy(), expect, **BF16)


@pytest.mark.parametrize("rows,cols,variant,split", [
    (2048, 16384, "split", 2), (2048, 16384, "split", 8),
    (512, 131072, "auto", 0),   # the forward group pipeline, 8 members
])
def test_rmsnorm_fwd_back_to_back(gpu, rows, cols, variant, split):
    x, w, _ = WORKLOADS["rmsnorm_bwd"].make_inputs(rows, cols, seed=7)
    xs, ws_ = x.to(gpu), w.to(gpu)
    y = torch.empty_like(xs)
    rstd = torch.empty(x.shape[0], device=gpu)
    cfg = hip_lib.make_cfg(variant, split)
    print(f"rmsnorm_fwd {variant} {split} ({rows}, {cols})", flush=True)
    queue(lambda: hip_lib.rmsnorm_fwd(xs, ws_, y, rstd, 1e-6, cfg))
    ey, er = ref.rmsnorm_fwd(x.float().numpy(), w.float().numpy(), 1e-6)
    np.testing.assert_allclose(rstd.cpu().numpy(), er, **FP32)
    np.testing.assert_allclose(y.float().cpu().numpy(), ey, **BF16)


def test_control_overhead_runs_clean(gpu):
    """The barrier microbenchmark takes the same co-resident shape."""
    plain_ms, split_ms = hip_lib.control_overhead(4096, 8, 2, warmup=2, iters=5)
    assert plain_ms > 0 and split_ms > 0


def test_split_calls_on_two_streams_use_their_own_workspaces(gpu):
    """NULL-workspace split calls on a second stream get that stream's own
    buffer (allocated and zeroed on first use) and the same results; the
    calls are serialised, so their grids never share the device."""
    x, w, dy = WORKLOADS["rmsnorm_fwd"].make_inputs(64, 65536, seed=8)
    xs, ws_ = x.to(gpu), w.to(gpu)
    results = []
    for stream in (torch.cuda.current_stream(), torch.cuda.Stream()):
        with torch.cuda.stream(stream):
            y, rstd = hip_lib.allocate_outputs("rmsnorm_fwd", (xs, ws_))
            hip_lib.rmsnorm_fwd(xs, ws_, y, rstd, 1e-6, hip_lib.make_cfg("split", 4))
            hip_lib.check_watchdog(hip_lib.make_cfg())
        stream.synchronize()
        results.append((y.cpu(), rstd.cpu()))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
