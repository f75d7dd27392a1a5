"""Device choice and budget on the host (internal/gpu/device.go:185-201
Best, internal/llm/service.go:210-212 DeviceBytes), over synthetic device
lists, and the rk_device_info layout the library fills."""
import ctypes

import rkhip


def info(index, memory, exact=1, integrated=0):
    d = rkhip.DeviceInfo()
    d.index, d.memory, d.exact, d.integrated = index, memory, exact, integrated
    return d


def test_best_prefers_exact_discrete_with_most_memory():
    devs = [info(0, 64 << 30, integrated=1), info(1, 192 << 30), info(2, 288 << 30), info(3, 512 << 30, exact=0)]
    assert rkhip.best(devs).index == 2
    # ties keep the first; integrated only when no discrete one is exact
    assert rkhip.best([info(0, 8), info(1, 8)]).index == 0
    assert rkhip.best([info(0, 99, integrated=1), info(1, 9, exact=0)]).index == 0
    assert rkhip.best([info(0, 99, exact=0)]) is None
    assert rkhip.best([]) is None


def test_device_budget_is_85_percent_in_integers():
    assert rkhip.device_bytes_budget(info(0, 288 * 10**9)) == 288 * 10**9 // 100 * 85
    assert rkhip.device_bytes_budget(info(0, 199)) == 1 * 85  # integer division first, as the reference


def test_device_info_layout_matches_header():
    """rk.h: int32 index, char name[64], char arch[32], int64 memory, int32
    compute_units, exact, integrated."""
    f = {n: getattr(rkhip.DeviceInfo, n) for n, _ in rkhip.DeviceInfo._fields_}
    assert (f["index"].offset, f["name"].offset, f["arch"].offset, f["memory"].offset) == (0, 4, 68, 104)
    assert (f["compute_units"].offset, f["exact"].offset, f["integrated"].offset) == (112, 116, 120)
    assert ctypes.sizeof(rkhip.DeviceInfo) == 128
