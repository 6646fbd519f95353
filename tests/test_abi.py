"""The C-ABI library loads, exports every symbol include/credit.h declares, and
rejects bad arguments on the host with the documented status (no GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

from credit_amd import hip_lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "credit.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(credit_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_functions():
    names = declared_functions()
    assert "credit_row_sum_max_f32" in names
    assert len(names) >= 8


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_header():
    assert set(declared_functions()) <= set(hip_lib.SIGNATURES)


def test_status_strings(lib):
    for code, name in hip_lib.STATUS_NAMES.items():
        assert lib.credit_status_string(code).decode() == name


def test_version(lib):
    assert lib.credit_version().decode().startswith("credit-hip")


def _cfg(**kw):
    cfg = hip_lib.CreditCfg()
    for k, v in kw.items():
        setattr(cfg, k, v)
    return cfg


FAKE = 0x100000  # never dereferenced: every case fails validation first


@pytest.mark.parametrize(
    "args,status",
    [
        ((None, FAKE, FAKE, 4, 4), -1),
        ((FAKE, None, FAKE, 4, 4), -1),
        ((FAKE, FAKE, None, 4, 4), -1),
        ((FAKE, FAKE, FAKE, 4, 0), -2),
        ((FAKE, FAKE, FAKE, -1, 4), -2),
        ((FAKE + 2, FAKE, FAKE, 4, 4), -3),
    ],
)
def test_row_sum_max_rejects(lib, args, status):
    assert lib.credit_row_sum_max_f32(*args, None) == status
    assert lib.credit_last_error().decode()


@pytest.mark.parametrize(
    "cfg,status",
    [
        (dict(variant=9), -8),
        (dict(split=-1), -8),
        (dict(split=65), -8),
        (dict(workspace=FAKE + 16), -5),
    ],
)
def test_bad_config_rejected(lib, cfg, status):
    c = _cfg(**cfg)
    assert lib.credit_row_sum_max_f32(FAKE, FAKE, FAKE, 4, 4, ctypes.byref(c)) == status


def test_layernorm_rejects(lib):
    args = [FAKE] * 6
    for i in range(6):
        bad = list(args)
        bad[i] = None
        assert lib.credit_layernorm_fwd_bf16(*bad, 4, 8, 1e-5, None) == -1
    assert lib.credit_layernorm_fwd_bf16(*args, 4, 0, 1e-5, None) == -2
    assert lib.credit_layernorm_fwd_bf16(*args, 4, 8, -1.0, None) == -8
    assert lib.credit_layernorm_fwd_bf16(*args, 4, 8, float("nan"), None) == -8


def test_rows_zero_is_a_noop(lib):
    assert lib.credit_row_sum_max_f32(FAKE, FAKE, FAKE, 0, 16, None) == 0


def test_workspace_bytes(lib):
    # READ needs none; SPLIT needs per-row partials plus the header.
    assert hip_lib.workspace_bytes("row_sum_max", 1024, 65536, "read") == 0
    ws = hip_lib.workspace_bytes("row_sum_max", 1024, 65536, "split", 4)
    assert ws >= 256 + 1024 * 4 * (8 + 4) + 1024 * 4
    assert hip_lib.workspace_bytes("row_sum_max", 0, 65536, "split", 4) == 0


def test_query_device_without_gpu_fails_cleanly(lib):
    info = hip_lib.DeviceInfo()
    assert lib.credit_query_device(-1, ctypes.byref(info)) == -8
    assert lib.credit_query_device(0, None) == -1


def test_bind_records_per_thread_and_replays_statuses(lib):
    """hip_lib.bind records a launcher's library calls (each reports OK while
    recording) and replays them, raising on a failing status; another thread
    sees the real library meanwhile.  No GPU: the replayed call fails
    argument validation, which runs before any HIP call."""
    import threading

    from credit_amd import hip_lib

    seen = {}

    def other_thread():
        seen["lib"] = hip_lib.load_library()

    def launcher(inputs, outputs, config):
        t = threading.Thread(target=other_thread)
        t.start()
        t.join()
        hip_lib.check(hip_lib.load_library().credit_row_sum_max_f32(None, None, None, 4, 4, None),
                      "credit_row_sum_max_f32")

    hip_lib.HIP_LAUNCHERS["_test_bind"] = launcher
    try:
        call = hip_lib.bind("_test_bind", (), ())
    finally:
        del hip_lib.HIP_LAUNCHERS["_test_bind"]
    assert seen["lib"] is hip_lib.load_library()
    assert not isinstance(hip_lib.load_library(), hip_lib._Recorder)
    with pytest.raises(hip_lib.CreditError) as err:
        call()
    assert err.value.status < 0
