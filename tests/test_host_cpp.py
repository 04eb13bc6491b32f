"""Builds (make -C tests/cpp) and runs the C++ tests of the vm_c host layer,
which exercise the block manager, layouts, metadata builder and error
convention without touching a GPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")


def test_host_layer_cpp():
    r = subprocess.run(["make", "-s", "-C", CPP, "_bin/test_host"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([os.path.join(CPP, "_bin", "test_host")], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
