"""The device-side exchange-tag sequence of split launches, through the C ABI.

Each split launch reads the workspace header's sequence word as it starts
and its last workgroup to exit advances it by the launch's stage count
(credit_amd/csrc/common.hpp, split_join / split_leave).  Checked here:
  - a split call captured into a HIP graph gives the eager call's outputs on
    every replay while its inputs change between replays (a tag fixed at
    capture time would let a replay take the previous replay's partials);
  - the sequence advances by exactly the launch's stages, and the launch
    that takes it past its limit returns the slot area to zero: slots planted
    with the tags the next launch polls for are not taken for its partials;
  - the ticket subsets follow the sizing rule (no group spans every slot of
    its subset) and workgroups are dealt to the XCDs round-robin.
"""
import ctypes

import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

SEQ_BYTE = 64           # header word of the tag sequence
# The row-ticket counter of the queued forward group pipeline: the counter
# area (256 bytes in, 262144 words) ends with its 64-byte line.
QUEUE_BYTE = 256 + 4 * (262144 - 16)
SLOT_OFFSET = 256 + (1 << 20)
SLOT_BYTES = 4 << 20
SEQ_LIMIT = 0xFFFFFFFF - (1 << 30)


def _seq(ws: torch.Tensor) -> int:
    return int(ws[SEQ_BYTE:SEQ_BYTE + 4].cpu().view(torch.int32).item()) & 0xFFFFFFFF


def _queue(ws: torch.Tensor) -> int:
    return int(ws[QUEUE_BYTE:QUEUE_BYTE + 4].cpu().view(torch.int32).item()) & 0xFFFFFFFF


def _set_seq(ws: torch.Tensor, value: int) -> None:
    v = np.array([value], dtype=np.uint32).view(np.uint8)
    ws[SEQ_BYTE:SEQ_BYTE + 4].copy_(torch.from_numpy(v.copy()))


def _softmax_bwd_inputs(rows, cols, seed, gpu):
    x, dy = (t.to(gpu) for t in WORKLOADS["softmax_bwd"].make_inputs(rows, cols, seed=seed))
    p, rowmax, lse = hip_lib.allocate_outputs("softmax_fwd", (x,))
    hip_lib.softmax_fwd(x, p, rowmax, lse, hip_lib.make_cfg())
    torch.cuda.synchronize()
    return p, dy


def _softmax_bwd(p, dy, cfg):
    dx = torch.full_like(p, float("nan"))
    hip_lib.softmax_bwd(p, dy, dx, cfg)
    return dx


def _workspace(op, rows, cols, gpu, variant="auto", split=0):
    nbytes = hip_lib.workspace_bytes(op, rows, cols, variant, split)
    assert nbytes > 0
    return torch.zeros(nbytes, dtype=torch.uint8, device=gpu)


def _expected_rows_per_group(rows, members):
    shape = hip_lib.last_split_shape()
    cus = hip_lib.query_device(0)["cu_count"]
    fit = shape["per_cu"] * cus // (8 * members) * 8
    padded = (rows + 7) // 8 * 8
    g = min(fit, padded)
    return -(-rows // g), shape


def test_graph_replays_of_a_group_kernel_follow_their_inputs(gpu):
    """softmax_bwd AUTO at 64 x 262144: the 32-member group kernel, captured
    once with a caller workspace, replayed with new dy each time."""
    rows, cols = 64, 262144
    print(f"softmax_bwd graph rows={rows} cols={cols}", flush=True)
    p, dy = _softmax_bwd_inputs(rows, cols, 21, gpu)
    ws = _workspace("softmax_bwd", rows, cols, gpu)
    dx = torch.empty_like(p)
    hip_lib.softmax_bwd(p, dy, dx, hip_lib.make_cfg(workspace=ws))  # eager warm-up
    torch.cuda.synchronize()
    rpg, shape = _expected_rows_per_group(rows, 32)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip_lib.softmax_bwd(p, dy, dx, hip_lib.make_cfg(workspace=ws))
    gen = torch.Generator().manual_seed(5)
    for replay in range(4):
        dy.copy_(torch.randn(rows, cols, generator=gen))
        before = _seq(ws)
        graph.replay()
        torch.cuda.synchronize()
        got = dx.clone()
        ref = _softmax_bwd(p, dy, hip_lib.make_cfg())
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {replay}"
        assert _seq(ws) == before + rpg
        hip_lib.check_watchdog(hip_lib.make_cfg(workspace=ws))
    del graph


def test_graph_replays_of_the_forward_group_pipeline(gpu):
    """rmsnorm_fwd AUTO at 64 x 131072: the forward group pipeline (8
    members), captured once with a caller workspace, replayed with new x."""
    rows, cols = 64, 131072
    print(f"rmsnorm_fwd graph rows={rows} cols={cols}", flush=True)
    x, w, _ = (t.to(gpu) for t in WORKLOADS["rmsnorm_fwd"].make_inputs(rows, cols, seed=13))
    ws = _workspace("rmsnorm_fwd", rows, cols, gpu)
    y, rstd = hip_lib.allocate_outputs("rmsnorm_fwd", (x, w))
    hip_lib.rmsnorm_fwd(x, w, y, rstd, hip_lib.RMSNORM_EPS, hip_lib.make_cfg(workspace=ws))
    torch.cuda.synchronize()
    _, shape = _expected_rows_per_group(rows, 8)
    assert shape["threads"] == 512 + 128  # data lanes, communication and ticket waves
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):  # the config takes the capture stream
        hip_lib.rmsnorm_fwd(x, w, y, rstd, hip_lib.RMSNORM_EPS, hip_lib.make_cfg(workspace=ws))
    gen = torch.Generator().manual_seed(6)
    for replay in range(4):
        x.copy_(torch.randn(rows, cols, generator=gen) * (1 + replay))
        before = _seq(ws)
        graph.replay()
        torch.cuda.synchronize()
        got = (y.clone(), rstd.clone())
        ry, rr = hip_lib.allocate_outputs("rmsnorm_fwd", (x, w))
        hip_lib.rmsnorm_fwd(x, w, ry, rr, hip_lib.RMSNORM_EPS, hip_lib.make_cfg())
        torch.cuda.synchronize()
        assert torch.equal(got[0], ry) and torch.equal(got[1], rr), f"replay {replay}"
        assert _seq(ws) == before + rows + 16  # a queued group may take every row
        assert _queue(ws) == 0, f"replay {replay}"
        hip_lib.check_watchdog(hip_lib.make_cfg(workspace=ws))
    del graph


def test_graph_replays_of_the_allocation_free_backward(gpu):
    """credit_rmsnorm_bwd_bf16_noalloc at 64 x 65536, split 8 (16 rows or
    fewer per group, inside the 16-row slot ring), captured once and
    replayed with new dy each time."""
    lib = hip_lib.load_library()
    rows, cols = 64, 65536
    print(f"rmsnorm_bwd_noalloc graph rows={rows} cols={cols}", flush=True)
    x, w, dy = (t.to(gpu) for t in WORKLOADS["rmsnorm_bwd"].make_inputs(rows, cols, seed=9))
    y, rstd = hip_lib.allocate_outputs("rmsnorm_fwd", (x, w))
    hip_lib.rmsnorm_fwd(x, w, y, rstd, hip_lib.RMSNORM_EPS, hip_lib.make_cfg())
    dx, dw = hip_lib.allocate_outputs("rmsnorm_bwd", (x, w, dy, rstd))

    def call():
        cfg = hip_lib.make_cfg("split", 8)
        hip_lib.check(lib.credit_rmsnorm_bwd_bf16_noalloc(
            x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
            dw.data_ptr(), rows, cols, ctypes.byref(cfg)), "credit_rmsnorm_bwd_bf16_noalloc")

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    gen = torch.Generator().manual_seed(6)
    for replay in range(4):
        dy.copy_(torch.randn(rows, cols, generator=gen).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = dx.clone(), dw.clone()
        rdx, rdw = hip_lib.allocate_outputs("rmsnorm_bwd", (x, w, dy, rstd))
        hip_lib.rmsnorm_bwd(x, w, dy, rstd, rdx, rdw, hip_lib.make_cfg("split", 8))
        torch.cuda.synchronize()
        assert torch.equal(got[0], rdx) and torch.equal(got[1], rdw), f"replay {replay}"
    hip_lib.check_watchdog()
    del graph


def test_sequence_wrap_clears_planted_slots(gpu):
    """A caller workspace whose sequence sits at its limit: the first launch
    (one row, so one group takes rows) tags its stages near 2^32 and its
    last workgroup returns the slot area to zero and the sequence to 0.  The
    slot area was planted beforehand with the tags the second launch polls
    for (stage s of every group and member: tag 1 + s, value 1e30), so a
    second launch that found them would finish with wrong dx at once."""
    rows, cols = 64, 262144
    print(f"softmax_bwd sequence wrap rows={rows} cols={cols}", flush=True)
    p, dy = _softmax_bwd_inputs(rows, cols, 31, gpu)
    ws = _workspace("softmax_bwd", rows, cols, gpu)
    members, ring = 32, 16
    words = SLOT_BYTES // 8
    idx = np.arange(words, dtype=np.uint64)
    tags = 1 + (idx // members) % ring
    planted = (tags << np.uint64(32)) | np.uint64(np.float32(1e30).view(np.uint32))
    ws[SLOT_OFFSET:SLOT_OFFSET + SLOT_BYTES].copy_(torch.from_numpy(planted.view(np.uint8)))
    _set_seq(ws, SEQ_LIMIT)
    one = _softmax_bwd(p[:1], dy[:1], hip_lib.make_cfg(workspace=ws))
    torch.cuda.synchronize()
    assert _seq(ws) == 0
    assert int(ws[SLOT_OFFSET:SLOT_OFFSET + SLOT_BYTES].count_nonzero()) == 0
    assert torch.equal(one, _softmax_bwd(p[:1], dy[:1], hip_lib.make_cfg()))
    got = _softmax_bwd(p, dy, hip_lib.make_cfg(workspace=ws))
    torch.cuda.synchronize()
    rpg, _ = _expected_rows_per_group(rows, members)
    assert _seq(ws) == rpg
    ref = _softmax_bwd(p, dy, hip_lib.make_cfg())
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    hip_lib.check_watchdog(hip_lib.make_cfg(workspace=ws))


def test_sequence_advances_by_each_launchs_stages(gpu):
    """softmax_fwd AUTO at 48 x 262144 (16-member group kernel): each call
    advances the caller workspace's sequence by its rows per group."""
    rows, cols = 48, 262144
    x = WORKLOADS["softmax_fwd"].make_inputs(rows, cols, seed=3)[0].to(gpu)
    ws = _workspace("softmax_fwd", rows, cols, gpu)
    p, rowmax, lse = hip_lib.allocate_outputs("softmax_fwd", (x,))
    seqs = []
    for _ in range(3):
        hip_lib.softmax_fwd(x, p, rowmax, lse, hip_lib.make_cfg(workspace=ws))
        torch.cuda.synchronize()
        seqs.append(_seq(ws))
    rpg, shape = _expected_rows_per_group(rows, 16)
    assert seqs == [rpg, 2 * rpg, 3 * rpg]
    assert shape["dispensers"] in (8, 4, 2, 1)
    hip_lib.check_watchdog(hip_lib.make_cfg(workspace=ws))


def test_ticket_subsets_hold_two_groups_and_xcc_dispatch_is_round_robin(gpu):
    """The split sizing rule (credit_amd/csrc/split_plan.hpp): every ticket
    subset's resident slots hold at least two groups.  C4 backward AUTO
    (32 members, one workgroup per CU) therefore takes four subsets of two
    XCDs each, C4 forward (16 members) eight.  The subsets follow the XCDs
    because workgroup b runs on XCC b % 8 (read from the hardware)."""
    info = hip_lib.query_device(0)
    n = info["xcd_count"]
    for grid in (256, 4096):
        xcc = [int(v) for v in hip_lib.microbench("xcc_map", n_results=grid)]
        print(f"xcc map of {grid} workgroups, first 48: {xcc[:48]}", flush=True)
        bad = [(b, v) for b, v in enumerate(xcc) if (v - xcc[0]) % n != b % n]
        print(f"  workgroups off the round-robin: {len(bad)}, first: {bad[:16]}", flush=True)
        assert sorted(set(xcc)) == list(range(n))
        assert not bad
    for name, rows, members in (("softmax_bwd", 16, 32), ("softmax_fwd", 16, 16)):
        cpu = WORKLOADS[name].make_inputs(rows, 262144, seed=1)
        ins = hip_lib.prepare_inputs(name, cpu, gpu)
        outs = hip_lib.allocate_outputs(name, ins)
        hip_lib.HIP_LAUNCHERS[name](ins, outs, hip_lib.LaunchConfig())
        torch.cuda.synchronize()
        shape = hip_lib.last_split_shape()
        resident = shape["per_cu"] * info["cu_count"]
        d = shape["dispensers"]
        assert resident // d >= 2 * members, (name, shape)
        assert d == 8 or resident // (2 * d) < 2 * members, (name, shape)
        if name == "softmax_bwd":
            assert d == 4 and shape["per_cu"] == 1, shape
    hip_lib.check_watchdog()


def test_query_device_fields(gpu):
    """credit_query_device on an MI355X: gfx950, 256 CUs in 8 XCDs (the
    runtime's XCC count), wave64, 160 KiB of LDS per CU and per workgroup
    (the FFN's 256-tile GEMM allocates all of it), 288 GB of HBM."""
    info = hip_lib.query_device(0)
    print(info, flush=True)
    assert info["arch"].startswith("gfx950")
    assert info["cu_count"] == 256 and info["xcd_count"] == 8
    assert info["wave_size"] == 64
    assert info["lds_bytes_per_cu"] == 160 * 1024
    assert info["lds_bytes_per_block"] == 160 * 1024
    assert info["l2_bytes"] >= 4 << 20
    assert info["hbm_bytes"] > 250 << 30


def test_control_overhead_takes_the_split_launchs_shape(gpu):
    """credit_control_overhead with the block size and LDS of the last split
    launch (credit_last_split_shape), as the runner passes them."""
    name, rows, cols = "softmax_bwd", 64, 262144
    ins = hip_lib.prepare_inputs(name, WORKLOADS[name].make_inputs(rows, cols, seed=2), gpu)
    outs = hip_lib.allocate_outputs(name, ins)
    hip_lib.HIP_LAUNCHERS[name](ins, outs, hip_lib.LaunchConfig())
    torch.cuda.synchronize()
    shape = hip_lib.last_split_shape()
    assert shape["threads"] == 512 + 64 and shape["per_cu"] == 1
    assert shape["lds_bytes"] >= 128 * 1024
    lds = hip_lib.control_lds_bytes(shape, hip_lib.query_device(0)["lds_bytes_per_cu"])
    plain, split = hip_lib.control_overhead(rows, 32, 1, warmup=2, iters=5, lds_bytes=lds,
                                            threads=shape["threads"])
    assert 0 < plain < 1 and 0 < split < 5
    hip_lib.check_watchdog()


@pytest.mark.parametrize("rows", [1, 7, 64, 255, 256, 257, 300, 1024, 1500])
def test_forward_row_queue_returns_to_zero(gpu, rows):
    """rmsnorm_fwd AUTO at 131072 columns takes rows from a launch-wide
    ticket counter (one draw per row processed; the drawer of the last
    ticket resets it).  After every launch the counter reads zero, every row
    matches the oracle, and repeated launches give identical outputs
    whichever group took which row.  Row counts below, at and above the
    groups' fixed share (8 steps per group)."""
    from oracle import reference as ref

    cols = 131072
    print(f"rmsnorm_fwd queue rows={rows}", flush=True)
    xc, wc, _ = WORKLOADS["rmsnorm_fwd"].make_inputs(rows, cols, seed=rows)
    x, w = xc.to(gpu), wc.to(gpu)
    ws = _workspace("rmsnorm_fwd", rows, cols, gpu)
    y, rstd = hip_lib.allocate_outputs("rmsnorm_fwd", (x, w))
    first = None
    for call in range(3):
        y.fill_(float("nan"))
        rstd.fill_(float("nan"))
        hip_lib.rmsnorm_fwd(x, w, y, rstd, hip_lib.RMSNORM_EPS, hip_lib.make_cfg(workspace=ws))
        torch.cuda.synchronize()
        assert hip_lib.last_split_shape()["threads"] == 512 + 128
        assert _queue(ws) == 0, f"call {call}"
        got = (y.clone(), rstd.clone())
        if first is None:
            first = got
            ey, er = ref.rmsnorm_fwd(xc.float().numpy(), wc.float().numpy(),
                                     hip_lib.RMSNORM_EPS)
            np.testing.assert_allclose(got[1].cpu().numpy(), er, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(got[0].float().cpu().numpy(), ey, rtol=1e-2, atol=1e-2)
        else:
            assert torch.equal(got[0], first[0]) and torch.equal(got[1], first[1]), call
    hip_lib.check_watchdog(hip_lib.make_cfg(workspace=ws))
