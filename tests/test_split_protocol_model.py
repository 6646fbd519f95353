"""The split-row protocol on host threads (tests/cpp/split_protocol_model.cpp):
ticket subsets, co-resident sizing, tagged slot rings and the device-side
tag sequence, with the library's own integer rules
(credit_amd/csrc/split_plan.hpp).  No GPU.

Each scenario pairs the rule the library follows with the mistake it
replaces, and the mistake must fail:
  - a slot withheld from a launch stalls a group that spans every slot of
    its subset (the sizing the 64-member softmax backward had when its wait
    expired) and not one sized by plan::dispensers_for;
  - a slot ring of 2 DEPTH - 1 rows lets a publisher overwrite a slot a slow
    member has not polled; 2 DEPTH rows do not;
  - replays of a captured launch whose tags were fixed at capture take the
    previous replay's partials silently; the device-side sequence does not;
  - the wrapping launch must clear the slot area, or planted stale tags are
    taken for partials.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("needs g++")
    exe = tmp_path_factory.mktemp("model") / "split_protocol_model"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-pthread",
                    str(HERE / "cpp" / "split_protocol_model.cpp"), "-o", str(exe)], check=True)
    return exe


def run(model, scenario):
    out = subprocess.run([str(model), scenario], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    m = re.search(rf"{scenario}: watchdog=(\d+) wrong=(\d+) expired=(\d+) seq=(\d+)", out.stdout)
    assert m, out.stdout
    extra = dict(re.findall(r"(\w[\w ]*?)=(\d+)", out.stdout.split(f"{scenario}:")[0]))
    return dict(watchdog=int(m[1]), wrong=int(m[2]), expired=int(m[3]), seq=int(m[4]),
                **{k.strip(): int(v) for k, v in extra.items()})


def test_withheld_slot_stalls_the_old_sizing(model):
    r = run(model, "withheld_old")
    assert r["dispensers"] == 8 and r["groups"] == 8
    assert r["watchdog"] == 1 and r["expired"] > 0


def test_withheld_slot_is_absorbed_by_two_groups_per_subset(model):
    r = run(model, "withheld_new")
    assert r["dispensers"] == 4 and r["groups"] == 8
    assert r == {**r, "watchdog": 0, "wrong": 0, "expired": 0}
    assert r["seq"] == 8  # 64 rows over 8 groups: 8 stages


def test_random_start_order_and_a_late_pending_workgroup(model):
    r = run(model, "late_new")
    assert r["watchdog"] == 0 and r["wrong"] == 0 and r["expired"] == 0


def test_slot_ring_of_two_depth_rows_suffices(model):
    assert run(model, "ring_ok")["watchdog"] == 0
    short = run(model, "ring_short")
    assert short["watchdog"] == 1 and short["wrong"] == 0


def test_graph_replays_need_the_device_sequence(model):
    host = run(model, "replay_host")
    assert host["wrong"] > 0 and host["watchdog"] == 0  # silent: no wait expires
    dev = run(model, "replay_device")
    assert dev["wrong"] == 0 and dev["watchdog"] == 0 and dev["seq"] == 3 * 2


def test_sequence_wrap_clears_the_slot_area(model):
    r = run(model, "wrap")
    assert r["wrong"] == 0 and r["watchdog"] == 0 and r["seq after the wrapping launch"] == 0
    assert run(model, "wrap_noclear")["wrong"] > 0
