"""The library's host code under AddressSanitizer + UndefinedBehaviorSanitizer
and under ThreadSanitizer (tests/sanitize): the state-blob parser over every
truncation and seeded mutations of valid blobs, argument validation of the C
entry points, and concurrent calls from eight threads. Device code is built as
in the product; without a GPU the device entry points return before any
launch."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"


@pytest.mark.parametrize("kind", ["asan", "tsan"])
def test_host_code_under_sanitizer(kind):
    if not shutil.which("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    b = subprocess.run(["make", "-C", str(HERE), kind], capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stderr[-2000:]
    r = subprocess.run([str(HERE / "_build" / f"host_checks_{kind}")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "host checks ok" in r.stdout
