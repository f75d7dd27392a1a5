"""The device the reference's default choice would take on this machine
(internal/gpu/device.go:185-201 Best): MI355X is exact (gfx950 kernels,
denormals kept) and discrete."""
import pytest

import rkhip

pytestmark = pytest.mark.gpu


def test_best_is_an_exact_discrete_gfx950():
    devs = rkhip.devices()
    assert devs, "no device"
    b = rkhip.best(devs)
    assert b is not None and b.exact == 1 and b.integrated == 0
    assert b.arch.decode().startswith("gfx950")
    assert rkhip.device_bytes_budget(b) == b.memory // 100 * 85
