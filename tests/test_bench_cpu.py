"""bench.py's default run on the CPU: the driver's contract (one JSON line,
the C3 record with roofline and cpu_baseline, C2/C5/C4 sub-records with
theirs) checked with a stand-in for the library context, so that the
record-building code runs end to end without a GPU.  The stand-in only
returns shapes and timings; no number here is a measurement."""
import io
import json
import os
import sys
from contextlib import redirect_stdout

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "rfx-fuse_amd"))

torch = pytest.importorskip("torch")


class _Event:
    def __init__(self, enable_timing=False):
        self.t = 0.0

    def record(self, stream=None):
        import time

        self.t = time.perf_counter()

    def elapsed_time(self, other):
        return max((other.t - self.t) * 1e3, 1e-3)


class _FakeContext:
    """Answers the calls bench.py makes, with tensors of the right shapes."""
    fail_on = None  # method name that raises (failure-path test)

    def __init__(self, device=0):
        self.n = 0

    def _maybe_fail(self, name):
        if _FakeContext.fail_on == name:
            raise RuntimeError(f"stand-in failure in {name}")

    def use_torch_stream(self):
        pass

    def set_forest(self, leaf, words, n, t, nleaf, layout="tree", nout=None):
        self._maybe_fail("set_forest")
        self.n = n

    def upper(self, fmt, out, r0=0, r1=None, scale=1.0, zp=0.0):
        pass

    def set_timing(self, on):
        pass

    def reset_timing(self):
        pass

    def kernel_time(self, name):
        return 0.5, 2

    def upper_recounts(self):
        return 0

    def upper_minmax(self, r0=0, r1=None):
        return 0.0, 1.0

    def set_reference(self, leaf, n, t, nleaf, layout="tree"):
        self._maybe_fail("set_reference")
        self.n = n

    def topk(self, qleaf, k, **kw):
        q = qleaf.shape[0]
        return torch.zeros((q, k), dtype=torch.int32), torch.zeros((q, k), dtype=torch.int16)

    def lowrank_pv(self, V):
        self._maybe_fail("lowrank_pv")
        return torch.empty_like(V)

    def lowrank_subspace(self, V0, iters):
        r = V0.shape[1]
        return torch.empty_like(V0), np.eye(r)

    def close(self):
        pass


@pytest.fixture
def cpu_bench(monkeypatch):
    import bench
    import rfxprox as R

    real_device = torch.device
    monkeypatch.setattr(torch, "device", lambda *a, **k: real_device("cpu"))
    monkeypatch.setattr(torch.cuda, "Event", _Event)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "init", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda *a, **k: None)
    monkeypatch.setattr(R, "Context", _FakeContext)
    small = {
        "c3": dict(bench.CONFIGS["c3"], n=3000, t=40, nleaf=64, leaves=(64, 64)),
        "c2": dict(bench.CONFIGS["c2"], n=2000, t=40, nleaf=64, leaves=(20, 64)),
        "c5": dict(bench.CONFIGS["c5"], n=4000, q=64, t=24, nleaf=32),
        "c4": dict(bench.CONFIGS["c4"], n=3000, t=20, nleaf=64, r=8),
        "cs2": dict(bench.CONFIGS["cs2"], n=300, t=6, nleaf=12),
    }
    monkeypatch.setattr(bench, "CONFIGS", small)
    _FakeContext.fail_on = None
    yield bench
    _FakeContext.fail_on = None


def _run(bench, argv):
    old = sys.argv
    sys.argv = ["bench.py"] + argv
    buf = io.StringIO()
    try:
        with redirect_stdout(buf):
            bench.main()
    finally:
        sys.argv = old
    lines = [ln for ln in buf.getvalue().splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    return json.loads(lines[0])


def test_default_run_prints_one_line_with_sub_records(cpu_bench):
    rec = _run(cpu_bench, ["--steps", "2", "--warmup", "1", "--cpu-seconds", "0.4"])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in rec, key
    assert rec["n_gpus"] == 1 and rec["steps"] == 2 and rec["dtype"] == "u8"
    roof = rec["roofline"]
    n, t = 3000, 40
    # compulsory bytes: output, int32 leaves, OOB bits, nout
    assert roof["compulsory_bytes"] == n * (n + 1) // 2 + n * t * 4 + n * t // 8 + n * 4
    for key in ("frac", "frac_compulsory_kernel", "frac_compulsory_step"):
        assert roof[key] > 0
    assert rec["cpu_baseline"]["kind"] == "port" and rec["cpu_baseline"]["value"] > 0
    # the quantizer rule on the data: min 0 / max 1 give the parameters used
    assert rec["quantizer"]["matches_the_scale_used"] is True
    subs = rec["sub_records"]
    assert set(subs) == {"c2", "c5", "c4"}
    for name, sub in subs.items():
        assert "error" not in sub, (name, sub)
        assert sub["value"] > 0 and sub["ms_per_step"] > 0
        assert sub["roofline"]["compulsory_bytes"] > 0 and sub["roofline"]["frac_compulsory_step"] > 0
        assert sub["cpu_baseline"]["value"] > 0
    assert subs["c2"]["dtype"] == "f32"


def test_a_failing_sub_record_does_not_stop_the_line(cpu_bench):
    _FakeContext.fail_on = "lowrank_pv"
    rec = _run(cpu_bench, ["--steps", "1", "--warmup", "1", "--no-cpu-baseline"])
    assert rec["value"] > 0
    assert "stand-in failure" in rec["sub_records"]["c4"]["error"]
    assert "error" not in rec["sub_records"]["c5"]


def test_single_config_and_no_sub(cpu_bench):
    rec = _run(cpu_bench, ["--config", "c5", "--steps", "1", "--warmup", "1", "--no-cpu-baseline"])
    assert "sub_records" not in rec and rec["config"]["Q"] == 64
    rec = _run(cpu_bench, ["--no-sub", "--steps", "1", "--warmup", "1", "--no-cpu-baseline"])
    assert "sub_records" not in rec and rec["dtype"] == "u8"


def test_more_than_one_gpu_exits(cpu_bench):
    old = sys.argv
    sys.argv = ["bench.py", "--gpus", "2"]
    buf = io.StringIO()
    try:
        with redirect_stdout(buf), pytest.raises(SystemExit) as e:
            cpu_bench.main()
    finally:
        sys.argv = old
    assert e.value.code == 2
    assert "one GPU" in json.loads(buf.getvalue())["error"]


def test_cs2_record_from_the_emulated_driver(cpu_bench, emu_driver, monkeypatch):
    """--config cs2 runs the class driver in its measure mode and turns its
    output into the record: here the driver is the one linked against the
    CPU emulation of the library (tests/emu), on a small forest."""
    monkeypatch.setattr(cpu_bench, "LRDRIVER", os.path.join(os.path.dirname(emu_driver), "lowrank_driver"))
    monkeypatch.setenv("ASAN_OPTIONS", "detect_stack_use_after_return=0:detect_leaks=0:abort_on_error=1")
    monkeypatch.setenv("EMU_TRACK_HOST", "1")
    rec = _run(cpu_bench, ["--config", "cs2"])
    assert rec["config"]["N"] == 300 and rec["config"]["rank"] == 17 and rec["steps"] == 6
    assert rec["ms_per_step"] > 0 and rec["value"] > 0 and rec["finalize_ms"] > 0
    assert rec["roofline"]["compulsory_bytes"] == 2 * 2 * (300 * 301 // 2)
    assert rec["device_bytes_after_add"]["max"] > 0
    assert rec["get_memory_usage"][1] == 2 * 300 * 17 * 2    # FP16 factors A and B
