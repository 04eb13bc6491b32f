"""Runs the GPU test of the vm_c host layer (tests/cpp/test_host_gpu.cpp,
built by __graft_entry__.build()): KVCacheManager pools, the metadata
builder and both attention backends end to end, against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_bin", "test_host_gpu")


def test_host_layer_on_gpu(dev):
    assert os.path.exists(BIN), "tests/cpp/_bin/test_host_gpu not built: run __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout and r.stdout.strip().endswith("ok")
