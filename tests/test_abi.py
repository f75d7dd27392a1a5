"""The C-ABI library loads and exports what include/rk.h declares (CPU:
no compute calls), and the Python bindings cover every entry point."""
import ctypes
import os
import re
import subprocess

import pytest

import rkhip


def header_functions(path=None):
    src = open(path or rkhip.HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(rk_\w+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_symbol():
    L = rkhip.lib()
    names = header_functions()
    assert len(names) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", rkhip.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (rk_\w+)$", out.stdout, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(L, n)


def test_bindings_cover_the_header():
    assert sorted(rkhip.SIGNATURES) == header_functions()


def test_worker_library_exports_what_rk_worker_h_declares():
    """librkworker.so (the tensor broker's worker side, host code only)
    against include/rk_worker.h, and its bindings (rkworker.py)."""
    import rkworker

    names = header_functions(rkworker.HEADER)
    assert names == ["rk_tensor_call"]
    out = subprocess.run(["nm", "-D", "--defined-only", rkworker.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (rk_\w+)$", out.stdout, flags=re.M))
    assert set(names) <= exported
    assert sorted(rkworker.SIGNATURES) == names
    for n in names:
        getattr(rkworker.lib(), n)


def test_no_device_is_an_error_not_a_crash():
    if rkhip.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(rkhip.RKError) as e:
        rkhip.Device(0)
    assert e.value.code == rkhip.RK_ERR_NO_DEVICE


def test_null_arguments_are_rejected():
    L = rkhip.lib()
    assert L.rk_device_count(None) == rkhip.RK_ERR_ARGS
    assert L.rk_device_open(0, None) == rkhip.RK_ERR_ARGS
    assert L.rk_device_close(None) == rkhip.RK_ERR_ARGS
    assert L.rk_used_bytes(None) == -1
    assert L.rk_matrix_free(None) == rkhip.RK_ERR_ARGS
    assert L.rk_matrix_bytes(None) == -1
    assert L.rk_matvecs(None, 0, None, None, None, 0) == rkhip.RK_ERR_ARGS
