"""Shared test setup: import paths for the product package and the oracle,
and the `gpu` marker (tests that need an MI355X)."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "rfx-fuse_amd"), os.path.join(REPO, "oracle"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (gfx950 / MI355X)")


@pytest.fixture(scope="session")
def gpu_ctx():
    """A librfxprox context on cuda:0.  GPU tests fail (not skip) when the
    device or the library is missing: there is no fallback path."""
    import torch

    import rfxprox

    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    torch.cuda.init()
    ctx = rfxprox.Context(0)
    ctx.use_torch_stream()
    yield ctx
    ctx.close()


@pytest.fixture(scope="session")
def emu_driver():
    """The CPU emulation build of the library (tests/emu/_build/emu_driver),
    made once per session; skipped where ROCm's host clang++ is absent."""
    import subprocess

    if not os.path.exists("/opt/rocm/llvm/bin/clang++"):
        pytest.skip("host clang++ of ROCm not present")
    emu = os.path.join(REPO, "tests", "emu")
    r = subprocess.run(["make", "-C", emu, "-j8"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    return os.path.join(emu, "_build", "emu_driver")
