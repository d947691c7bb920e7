"""The C ABI from a compiled C++ caller (tests/c_abi/test_abi_c.cpp): hipMalloc'd
buffers, a hand-uploaded grouped table and a caller workspace, no torch in the
process; every result compared byte for byte with the CPU oracle."""

from __future__ import annotations

import os
import subprocess

import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "c_abi", "_build", "test_abi_c")


@pytest.mark.gpu
def test_c_caller_matches_oracle():
    assert os.path.exists(BIN), f"{BIN} is not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=180)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "c-abi ok" in r.stdout
