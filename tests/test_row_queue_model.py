"""The row-ticket queue of the group pipelines on host threads
(tests/cpp/row_queue_model.cpp): one thread per row group drawing tickets
from one atomic counter at random rates, with the rules of
credit_amd/csrc/common.hpp (queue_ticket_wave, queue_take_row).  No GPU.

Back-to-back launches on one counter must each process every row exactly
once and leave the counter at zero.  Two planted mistakes must fail: the
reset left out, and one extra draw after a group's last stage (the count of
draws per launch is what makes the drawer of value rows - 1 the last one).
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
    exe = tmp_path_factory.mktemp("queue") / "row_queue_model"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-pthread",
                    str(HERE / "cpp" / "row_queue_model.cpp"), "-o", str(exe)], check=True)
    return exe


def run(model, scenario):
    out = subprocess.run([str(model), scenario], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    m = re.search(rf"{scenario}: launches=(\d+) wrong=(\d+) dup=(\d+) counter=(\d+)", out.stdout)
    assert m, out.stdout + out.stderr
    assert "out of range" not in out.stderr, out.stderr
    return dict(launches=int(m[1]), wrong=int(m[2]), dup=int(m[3]), counter=int(m[4]))


def test_every_row_once_and_the_counter_back_at_zero(model):
    r = run(model, "queue")
    assert r == {"launches": 30, "wrong": 0, "dup": 0, "counter": 0}


def test_without_the_reset_later_launches_lose_rows(model):
    r = run(model, "no_reset")
    assert r["wrong"] > 0 and r["counter"] != 0


def test_an_extra_draw_leaves_the_counter_off_zero(model):
    r = run(model, "extra_draw")
    assert r["counter"] != 0 and r["wrong"] > 0
