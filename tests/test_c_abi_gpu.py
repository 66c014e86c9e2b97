"""The C ABI used from C++ without Python or torch (tests/c/abi_roundtrip.cpp,
built by daser_amd._build), run as a child process on the GPU."""

import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "abi_roundtrip")


@pytest.mark.gpu
def test_c_abi_round_trip(gpu):
    print("case: C ABI round trip", flush=True)
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run python -m daser_amd._build")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_roundtrip ok" in r.stdout
