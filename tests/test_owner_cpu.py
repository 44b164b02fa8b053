"""CPU check of the claim that keeps a context or batch to one host thread at
a time (needle-rs_amd/csrc/nd_owner.h; entry points answer ND_ERR_BUSY when
another thread is inside a call on the object): built with the host compiler
and run, no GPU."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "needle-rs_amd", "csrc")


def test_owner_claim_is_exclusive_and_reentrant(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = str(tmp_path / "owner_check")
    subprocess.run([gxx, "-O2", "-std=c++17", "-pthread", "-I", CSRC, "-o", out,
                    os.path.join(HERE, "owner_check.cpp")], check=True)
    r = subprocess.run([out], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
