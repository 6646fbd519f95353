"""The gfx950 calibration microbenchmarks on the GPU: what the cost model
and the bench's stream ceilings consume must be physically ordered and at
least what the library's own kernels reach."""
import math

import pytest
import torch

from credit_amd import hip_lib
from credit_amd.timing import run_trials
from credit_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu


def test_latency_chain_is_ordered(gpu):
    lat = hip_lib.microbench("latency", 0, 20000, 4)
    print(f"latency cycles L1/L2/MALL/HBM: {lat[:4]}", flush=True)
    assert all(math.isfinite(v) and v > 0 for v in lat[:4])
    assert lat[0] < lat[1] < lat[2] < lat[3]


def test_cache_and_exchange_throughput(gpu):
    l1, l2_xcd, l2_gbps = hip_lib.microbench("cache_read", 0, 64, 3)
    print(f"L1 {l1:.1f} B/cycle/CU, L2 {l2_xcd:.1f} B/cycle/XCD = {l2_gbps:.0f} GB/s", flush=True)
    # Physically bounded: an L1 returns at most a few hundred bytes per cycle
    # per CU, an XCD's L2 (16 channels of 128 B) at most ~4 KiB per cycle,
    # and L2 hits come faster than HBM's 8 TB/s peak.
    assert 8 < l1 < 512
    assert 0 < l2_xcd < 4096 and l2_gbps > 8000.0
    store, store_gbps, tick_private, tick_shared = hip_lib.microbench(
        "exchange_throughput", 0, 4096, 4)
    print(f"slot stores {store:.2f} B/cycle/WG ({store_gbps:.0f} GB/s), ticket draws "
          f"{tick_private:.0f} / {tick_shared:.0f} cycles", flush=True)
    assert store > 0 and store_gbps > 0
    assert 0 < tick_private < tick_shared  # one line for every CU serialises
    rt = hip_lib.microbench("exchange_roundtrip", 0, 2000, 2)
    assert all(math.isfinite(v) and v > 0 for v in rt[:2])


def test_stream_read_ceiling_covers_the_row_reduction(gpu):
    """The calibration's HBM read stream must reach at least what C1's row
    kernel reaches on the same bytes (timed the same way), or the cost
    model's bandwidth term is biased low."""
    spec = WORKLOADS["row_sum_max"]
    nbytes = spec.algorithmic_bytes(spec.rows, spec.cols)
    sets = [hip_lib.prepare_inputs("row_sum_max", spec.make_inputs(), gpu) for _ in range(3)]
    outs = [hip_lib.allocate_outputs("row_sum_max", s) for s in sets]
    calls = [hip_lib.bind("row_sum_max", s, o) for s, o in zip(sets, outs)]
    t = run_trials(lambda i: calls[i % 3](), 5, 20, warmup=5, settle_ms=100.0)
    kernel_gbps = nbytes / (t.median_ms * 1e-3) / 1e9
    ceiling = hip_lib.stream_ceiling(1, 0, nbytes)
    print(f"C1 {kernel_gbps:.0f} GB/s, read ceiling {ceiling}", flush=True)
    assert ceiling["GBps"] >= 0.97 * kernel_gbps
    assert ceiling["GBps"] < 8000.0 * 1.05  # cannot beat the HBM peak by more than noise
    del sets, outs, calls
    torch.cuda.empty_cache()


def test_stream_ceiling_rejects_unbuilt_mixes(gpu):
    with pytest.raises(hip_lib.CreditError):
        hip_lib.stream_ceiling(3, 3, 1 << 26)
    with pytest.raises(hip_lib.CreditError):
        hip_lib.stream_ceiling(1, 1, 1024)  # under 64 KiB per stream


def test_mfma_rate_is_physical(gpu):
    """The MFMA rate the FFN is compared with: positive, at most the
    datasheet 2.5 PFLOP/s (plus noise), and per shader cycle at most the
    4 SIMDs x 1024 flops a CU's matrix cores issue."""
    c = hip_lib.mfma_ceiling(4000)
    print(f"MFMA bf16 {c}", flush=True)
    assert 500.0 < c["TFLOPs"] < 2500.0 * 1.05
    assert 500.0 < c["clock_MHz"] < 3000.0
    assert c["flops_per_cycle_cu"] < 4096 * 1.05
