"""Device self-check of MFMA layouts and lane-level reductions (runs first:
every kernel's correctness rests on these)."""
import pytest

pytestmark = pytest.mark.gpu


def test_selftest(dev):
    from vm_c_amd import capi
    capi.selftest()
