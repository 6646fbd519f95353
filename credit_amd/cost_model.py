"""Split-row cost model recalibrated for gfx950 (CDNA4).

The reference's model (dsmem_eval/cost_model.py:62-141) predicts whether a
thread-block-cluster variant that stages a 1/P row slice per CTA in shared
memory and exchanges partials through DSMEM beats the best one-CTA-per-row
variant:

    delta = saved_reread - control - local_replay - local_store_residual
            - dsmem_store                                   (:125-131)

with ``effective bandwidth`` taken from the measured baseline (:79-82).
CDNA4 has no DSMEM.  The split variant here stages its slice on chip
(VGPRs, spilling to LDS) and its P workgroups meet at arrival barriers in an
L2-resident workspace.  The terms become:

* ``saved_reread_ms``  -- as the reference (:83-87), but only when the
  no-split variant actually re-reads HBM: a gfx950 workgroup holds up to
  ``onchip_bytes_per_workgroup`` (1024 lanes x 64 VGPRs plus the LDS
  allocation), so rows narrower than that are single-pass without a split
  and nothing is saved.
* ``fill_gain_ms``     -- new: a launch of ``rows`` one-per-row workgroups
  that keeps fewer bytes in flight than HBM latency x bandwidth needs runs
  latency-bound; splitting multiplies the workgroups in flight by P.  The
  gain is the baseline's latency-bound share that P more workgroups recover.
* ``control_overhead_ms`` -- measured: cooperative launch plus the arrival
  barriers, minus a plain launch (``credit_control_overhead``; the
  reference's cluster_control.cu).
* ``lds_replay_ms``    -- the staged slice re-read from LDS per extra pass
  (the reference's local_replay_ms, :100-108), charged only for the part of
  the slice that does not fit in VGPRs.
* ``l2_exchange_ms``   -- replaces dsmem_store_ms (:91-99): per wave of
  resident groups, one device-scope arrival and partial round trip per
  barrier, at the measured same-XCD atomic round trip.
* ``hidden_sync_ms``   -- new: the part of control + exchange a pipelined
  split kernel hides.  The group kernels publish a row's partial
  ``split_pipeline_depth`` row-steps before they need its total, so per row
  the exchange overlaps that many steps of streaming; the control overhead
  is measured with the exchanges back to back (credit_control_overhead, at
  the launch's own block size and LDS), so it is charged only beyond
  depth x the compulsory stream time.  0 for the barrier-synchronised slice
  kernels.  The depth is the one of the kernel the split runs (v3: per
  split factor, from the workload's planner rules; v2 had one depth per
  workload).

``estimate()`` keeps the reference's signature and result shape so the
runner's summary logic (dsmem_eval/runner.py:444-620) carries over.

``predict_traffic()`` states the bytes behind those terms -- HBM bytes of
the split and of the best no-split variant, L2 requests of the split and the
LDS bytes its exchange and replay move -- so a sweep can put hardware
counters (credit_amd.counters) beside them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Protocol


class WorkloadModelSpec(Protocol):
    rows: int
    modeled_bytes_per_element: float
    reread_bytes_per_element: float
    staged_bytes_per_element: int
    partial_count: int
    barrier_count: int


MODEL_VERSION = "cdna4-onchip-fill-exchange-v3"

# Register staging budget of one 1024-lane workgroup: 64 VGPRs of data per
# lane (the rest of the 512-entry file holds addresses and accumulators).
REGISTER_STAGING_BYTES = 1024 * 64 * 4
# Bytes one lane keeps in flight in the streaming kernels (8 dwordx4 loads).
INFLIGHT_BYTES_PER_LANE = 8 * 16
# Lanes a no-split streaming workgroup runs (one row per workgroup).
STREAM_LANES_PER_WORKGROUP = 256
# Workgroups of that size resident per CU (VGPR-limited at ~64 VGPRs).
STREAM_WORKGROUPS_PER_CU = 8


@dataclass(frozen=True)
class DeviceProfile:
    """Measured gfx950 figures (credit_amd.profile.make_device_profile)."""

    name: str
    cu_count: int
    xcd_count: int
    clock_ghz: float
    hbm_read_gbps: float
    hbm_copy_gbps: float
    l2_capacity_bytes: int
    lds_bytes_per_cu: int
    max_lds_bytes_per_block: int
    lds_read_bytes_per_cycle_cu: float
    lds_write_bytes_per_cycle_cu: float
    exchange_roundtrip_cycles: float
    hbm_latency_cycles: float

    @property
    def onchip_bytes_per_workgroup(self) -> int:
        return REGISTER_STAGING_BYTES + self.max_lds_bytes_per_block


# Nominal MI355X figures, used where no calibration has been run (CPU tests,
# offline re-scoring of saved results).
MI355X_NOMINAL = DeviceProfile(
    name="MI355X (nominal)",
    cu_count=256,
    xcd_count=8,
    clock_ghz=2.4,
    hbm_read_gbps=8000.0,
    hbm_copy_gbps=8000.0,
    l2_capacity_bytes=4 << 20,
    lds_bytes_per_cu=160 << 10,
    max_lds_bytes_per_block=160 << 10,
    lds_read_bytes_per_cycle_cu=128.0,
    lds_write_bytes_per_cycle_cu=128.0,
    exchange_roundtrip_cycles=2000.0,
    hbm_latency_cycles=2000.0,
)


@dataclass(frozen=True)
class ModelEstimate:
    effective_bandwidth_gbps: float
    saved_reread_ms: float
    fill_gain_ms: float
    control_overhead_ms: float
    lds_replay_ms: float
    l2_exchange_ms: float
    predicted_delta_ms: float
    predicted_profitable: bool
    hidden_sync_ms: float = 0.0

    @property
    def saved_hbm_ms(self) -> float:
        """Name of the saving in the reference's result bundles."""
        return self.saved_reread_ms

    @property
    def local_staging_ms(self) -> float:
        return self.lds_replay_ms


def staged_bytes_per_workgroup(spec: WorkloadModelSpec, cols: int, split: int) -> int:
    """On-chip bytes one member holds (shared_bytes_per_cta of
    dsmem_eval/cost_model.py:55-60)."""
    return math.ceil(cols / split) * spec.staged_bytes_per_element


def row_fits_one_workgroup(spec: WorkloadModelSpec, cols: int, profile: DeviceProfile) -> bool:
    """Whether the no-split variant holds the row on chip (single HBM pass):
    the kernel's own STAGED capacity when the spec states it, else the
    VGPR + LDS budget of one workgroup."""
    cap = getattr(spec, "staged_max_cols", 0)
    if cap:
        return cols <= cap
    return staged_bytes_per_workgroup(spec, cols, 1) <= profile.onchip_bytes_per_workgroup


def fill_fraction(workgroups: int, lanes: int, profile: DeviceProfile) -> float:
    """Share of peak HBM bandwidth a grid of `workgroups` streaming
    workgroups can sustain by Little's law: bytes in flight over
    bandwidth x latency."""
    resident = min(workgroups, profile.cu_count * STREAM_WORKGROUPS_PER_CU * 256 // max(lanes, 1))
    inflight = resident * lanes * INFLIGHT_BYTES_PER_LANE
    latency_s = profile.hbm_latency_cycles / (profile.clock_ghz * 1e9)
    need = profile.hbm_read_gbps * 1e9 * latency_s
    return min(1.0, inflight / need) if need > 0 else 1.0


def estimate(
    spec: WorkloadModelSpec,
    cols: int,
    cluster_size: int,
    control_overhead_ms: float,
    profile: DeviceProfile,
    baseline_ms: float,
    rows: int | None = None,
) -> ModelEstimate:
    """Predicted gain of the P-way split over the measured no-split time.

    Same signature as dsmem_eval/cost_model.py:62-70 (``cluster_size`` is
    the split factor P)."""
    row_count = spec.rows if rows is None else rows
    split = int(cluster_size)
    if split < 2:
        raise ValueError("cluster_size (split) must be >= 2")
    if not math.isfinite(baseline_ms) or baseline_ms <= 0.0:
        raise ValueError("baseline_ms must be finite and positive")
    if spec.modeled_bytes_per_element <= 0.0:
        raise ValueError("modeled_bytes_per_element must be positive")

    modeled = row_count * cols * spec.modeled_bytes_per_element
    effective_bandwidth_gbps = modeled / (baseline_ms * 1.0e6)

    single_pass = row_fits_one_workgroup(spec, cols, profile)
    if single_pass:
        saved_reread_ms = 0.0
        remaining_ms = baseline_ms
    else:
        saved_reread_ms = baseline_ms * spec.reread_bytes_per_element / spec.modeled_bytes_per_element
        remaining_ms = baseline_ms - saved_reread_ms

    # Latency-bound share of the remaining (compulsory) stream.
    lanes = 1024 if single_pass else STREAM_LANES_PER_WORKGROUP
    fill_nosplit = fill_fraction(row_count, lanes, profile)
    fill_split = fill_fraction(row_count * split, lanes, profile)
    fill_gain_ms = remaining_ms * (1.0 - fill_nosplit / fill_split) if fill_split > 0 else 0.0

    # Residency: groups of P members; every wave of groups pays the exchange.
    groups_resident = max(profile.cu_count * 2 // split, 1)
    waves = math.ceil(row_count / groups_resident)
    cycle_ms = 1.0 / (profile.clock_ghz * 1.0e6)
    l2_exchange_ms = waves * spec.barrier_count * profile.exchange_roundtrip_cycles * cycle_ms

    slice_bytes = staged_bytes_per_workgroup(spec, cols, split)
    spilled = max(slice_bytes - REGISTER_STAGING_BYTES, 0)
    extra_passes = max(spec.barrier_count - 1, 0)
    lds_replay_ms = (waves * spilled * extra_passes / profile.lds_read_bytes_per_cycle_cu) * cycle_ms

    control = max(control_overhead_ms, 0.0)
    depth = getattr(spec, "split_pipeline_depth", 0)
    if callable(depth):
        depth = depth(cols, split)
    hidden_sync_ms = min(control + l2_exchange_ms, depth * remaining_ms)
    delta = (saved_reread_ms + fill_gain_ms - (control + l2_exchange_ms - hidden_sync_ms)
             - lds_replay_ms)
    return ModelEstimate(
        effective_bandwidth_gbps=effective_bandwidth_gbps,
        saved_reread_ms=saved_reread_ms,
        fill_gain_ms=fill_gain_ms,
        control_overhead_ms=control,
        lds_replay_ms=lds_replay_ms,
        l2_exchange_ms=l2_exchange_ms,
        predicted_delta_ms=delta,
        predicted_profitable=delta > 0.0,
        hidden_sync_ms=hidden_sync_ms,
    )


# L2 request sizes the traffic prediction counts in: a wave's streaming
# read asks the L2 for whole 128-byte lines, its writes arrive as 64-byte
# requests (TCC_REQ of the read-only row reduction is its line count; of a
# 1:1 read:write stream, 1.5 times it).
L2_LINE_BYTES = 128
L2_WRITE_REQUEST_BYTES = 64


@dataclass(frozen=True)
class TrafficPrediction:
    hbm_bytes: float          # split variant: one HBM pass plus the exchange slots
    block_hbm_bytes: float    # best no-split variant: plus the re-read when the row does not fit
    l2_requests: float        # split variant: streamed reads and writes plus exchange traffic
    lds_bytes: float          # split variant: exchange copies plus the spilled-slice replay
    exchange_bytes: float     # split variant: slot stores and one poll per member and stage


def predict_traffic(spec, cols: int, split: int, profile: DeviceProfile,
                    rows: int | None = None) -> TrafficPrediction:
    """Bytes one call moves under the model's assumptions (the same ones
    estimate() prices): every member reads its slice once, so the split
    moves the algorithmic bytes; the no-split variant re-reads
    ``reread_bytes_per_element`` when the row does not fit one workgroup;
    every exchange stage costs each member one 8-byte slot store per
    partial and one poll of the group's slots (the minimum: a poll that
    finds a partial missing is repeated).  Slot stores and polls are
    device-scope accesses that pass the L2 to the memory side, so the HBM
    counters see them with the streamed bytes.  The exchanged values are
    copied once into each member's LDS; a slice beyond the register budget
    is replayed from LDS once per extra pass."""
    row_count = spec.rows if rows is None else rows
    p = int(split)
    compulsory = float(spec.algorithmic_bytes(row_count, cols))
    reads, writes = getattr(spec, "stream_mix", (1, 0))
    if reads + writes <= 0:
        reads, writes = 1, 0
    write_share = writes / (reads + writes)
    reread = 0.0 if row_fits_one_workgroup(spec, cols, profile) else \
        float(row_count) * cols * spec.reread_bytes_per_element
    k = max(int(spec.partial_count), 1)
    stages = float(row_count) * max(int(spec.barrier_count), 1)
    slot_bytes = stages * p * (8.0 * k + 8.0 * k * p)  # stores + one poll per member
    exchange_requests = stages * p * (k + math.ceil(8.0 * k * p / L2_LINE_BYTES))
    spilled = max(staged_bytes_per_workgroup(spec, cols, p) - REGISTER_STAGING_BYTES, 0)
    extra_passes = max(int(spec.barrier_count) - 1, 0)
    lds = stages * p * (4.0 * k * p) + float(row_count) * p * spilled * extra_passes
    return TrafficPrediction(
        hbm_bytes=compulsory + slot_bytes,
        block_hbm_bytes=compulsory + reread,
        l2_requests=(compulsory * (1.0 - write_share) / L2_LINE_BYTES +
                     compulsory * write_share / L2_WRITE_REQUEST_BYTES + exchange_requests),
        lds_bytes=lds,
        exchange_bytes=slot_bytes,
    )

