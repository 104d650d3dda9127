"""CPU-side checks of the product library: it loads, exports every function
that include/rfx_prox.h declares, its host-only helpers compute the right
sizes, and without a GPU it fails with an error instead of falling back."""
import ctypes
import os
import subprocess

import pytest

import rfxprox as R

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_function():
    lib = R.load()
    names = R.header_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", R.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    for n in R.header_functions():
        assert f" T {n}\n" in out + "\n" or f" T {n}" in out


def test_upper_nbytes():
    N = 100_000
    assert R.upper_nbytes(R.FMT_U8, N) == N * (N + 1) // 2 == 5_000_050_000
    assert R.upper_nbytes(R.FMT_F32, 20_000) == 4 * 200_010_000
    assert R.upper_nbytes(R.FMT_U16, 7) == 2 * 28
    # NF4: bytes touched by entries [e0, e1)
    assert R.upper_nbytes(R.FMT_NF4, 5) == 8          # 15 entries
    assert R.upper_nbytes(R.FMT_NF4, 5, 1, 3) == 4    # entries 5..11 -> bytes 2..5
    with pytest.raises(ValueError):
        R.upper_nbytes(R.FMT_U8, 10, 5, 4)
    with pytest.raises(ValueError):
        R.upper_nbytes(17, 10)


def test_no_device_is_an_error_not_a_fallback():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(R.RfxpError):
        R.Context(0)
    buf = ctypes.create_string_buffer(256)
    R.load().rfxp_last_error(None, buf, 256)
    assert b"no HIP device" in buf.value
