"""The library's per-(device, stream) workspace cache, checked on the host:
credit_amd/csrc/workspace_cache.hpp compiled with g++ against a recording
allocator (tests/cpp/workspace_cache_test.cpp).  No GPU."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_cache_keying_growth_and_retirement(tmp_path):
    exe = tmp_path / "workspace_cache_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-pthread",
                    str(HERE / "cpp" / "workspace_cache_test.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert "workspace cache: ok" in out.stdout
