"""The reference-signature layer in C++ (include/rfx_compat.hpp, the
LowRankProximityMatrix class, rfx::ForestProximity of
include/rfx_forest.hpp), driven by the same C++ programs as the GPU tests
(tests/compat/*_driver.cpp) but linked against the library built for the CPU
emulator (tests/emu), under AddressSanitizer.  The checks are the GPU tests'
own functions, run with the driver path pointed at the emulated build."""
import os

import pytest

import test_gpu_compat as GC
import test_gpu_forest_shim as GF
import test_gpu_lowrank_class as GL


@pytest.fixture
def emu_build(emu_driver, monkeypatch):
    monkeypatch.setenv("ASAN_OPTIONS", "detect_stack_use_after_return=0:detect_leaks=0:abort_on_error=1")
    monkeypatch.setenv("EMU_TRACK_HOST", "1")   # host pointers are host memory, as on a GPU
    return os.path.dirname(emu_driver)


@pytest.mark.parametrize("cw", [0, 1])
def test_reference_signatures(emu_build, monkeypatch, tmp_path, cw):
    monkeypatch.setattr(GC, "DRIVER", os.path.join(emu_build, "compat_driver"))
    GC.test_reference_signatures_through_cpp_driver(tmp_path, cw)


@pytest.mark.parametrize("n,nnode,t,cw,seed", GC.RANDOM_DRIVER_CASES)
def test_reference_signatures_on_random_forests(emu_build, monkeypatch, tmp_path, n, nnode, t, cw, seed):
    """Includes N*N odd, where the dense FP16 / INT8 / NF4 outputs of
    launch_proximity_kernel end inside a 32-bit word: the sanitizer sees any
    access past the output's last byte."""
    monkeypatch.setattr(GC, "DRIVER", os.path.join(emu_build, "compat_driver"))
    GC.check_random_forest_through_cpp_driver(tmp_path, n, nnode, t, cw, seed)


@pytest.mark.parametrize("level", [0, 1, 2, 3])
def test_lowrank_class_growtree_sequence(emu_build, monkeypatch, tmp_path, level):
    monkeypatch.setattr(GL, "LRDRIVER", os.path.join(emu_build, "lowrank_driver"))
    GL.test_class_growtree_sequence(tmp_path, level)


def test_lowrank_class_rfgap_sequence(emu_build, monkeypatch, tmp_path):
    monkeypatch.setattr(GL, "LRDRIVER", os.path.join(emu_build, "lowrank_driver"))
    GL.test_class_rfgap_sequence(tmp_path)


def test_forest_proximity_object(emu_build, monkeypatch, tmp_path):
    monkeypatch.setattr(GF, "FDRIVER", os.path.join(emu_build, "forest_driver"))
    GF.test_forest_proximity_object(tmp_path, 400, 37, 9, 23, 24)   # pairs past N = 400 read as out of range


def test_lowrank_class_growtree_sequence_through_the_dense_form(emu_build, monkeypatch, tmp_path):
    """The growtree sequence at N = 1,200 with 30 trees of 12 leaves, whose
    nonzeros pass the entry-list limit, so the accumulator changes to the
    dense triangle on the way; the GPU suite runs the same check at
    N = 5,000."""
    monkeypatch.setattr(GL, "LRDRIVER", os.path.join(emu_build, "lowrank_driver"))
    d = GL.check_growtree_at_scale(tmp_path, 1200, 30, 12, 1200, timeout=600)
    used = d["stats"]["used"]
    assert used[-1] == used[-2]   # the dense form holds no per-add memory
