"""Host-side unit tests of device helpers that also compile for the host."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "_build" / "fastdiv_test"


def test_fastdiv_matches_integer_division():
    if not BIN.exists():
        pytest.skip("tests/cpp not built (run __graft_entry__.build())")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 wrong" in r.stdout
