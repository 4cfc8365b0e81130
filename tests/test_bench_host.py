"""Host-side behaviour of bench.py (no device): the one-GPU contract, the order in which a group's
timed launches run, and the per-class summary arithmetic."""

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one MI355X" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


class _Event:
    """A stand-in event: elapsed time from a fixed table, in recording order."""

    def __init__(self, log):
        self.log = log
        self.t = None

    def record(self):
        self.t = len(self.log.records)
        self.log.records.append(self)

    def synchronize(self):
        pass

    def elapsed_ms(self, other):
        return self.log.ms[(other.t - 1) // 2]


class _Buffer:
    def __init__(self, nbytes):
        self.ptr = 0
        self.nbytes = nbytes


class _Hm:
    def __init__(self, ms=None):
        self.records = []
        self.ms = ms or [1.0] * 1000
        self.DeviceBuffer = _Buffer

    def Event(self):
        return _Event(self)

    def synchronize(self):
        pass


class _K:
    def __init__(self, calls):
        self.calls = calls

    def fill(self, ptr, elem, pattern, n):
        self.calls.append("fill")


def _run(order, monkeypatch):
    calls = []
    K, hm = _K(calls), _Hm()

    def builder(K_, hm_):
        work = [(lab, 100, 10, (lambda lab=lab: calls.append(lab))) for lab in ("a", "b", "c")]
        return work, []

    monkeypatch.setattr(bench, "CLASS_ORDER", order)
    out = bench.run_group(K, hm, builder)
    return calls, out


def test_classes_are_timed_as_blocks_by_default(monkeypatch):
    calls, out = _run(bench.CLASS_ORDER, monkeypatch)
    assert bench.CLASS_ORDER == "blocked"
    warm = ["a", "b", "c"] * bench.WARM
    timed = [x for lab in ("a", "b", "c") for x in ["fill", lab] * bench.TIMED]
    assert calls == warm + timed
    assert sorted(out) == ["a", "b", "c"] and all(v["launches"] == bench.TIMED for v in out.values())


def test_interleaved_order_kept_for_comparison(monkeypatch):
    calls, _ = _run("interleaved", monkeypatch)
    warm = ["a", "b", "c"] * bench.WARM
    timed = ["fill", "a", "fill", "b", "fill", "c"] * bench.TIMED
    assert calls == warm + timed


def test_timeline_summary_is_the_median_rate():
    ms = [0.5, 0.1, 0.3, 0.2, 0.4]  # median 0.3 ms
    hm = _Hm(ms)
    tl = bench.Timeline(hm)
    for _ in ms:
        tl.run("x", 8_000_000, 2_000_000, lambda: None)
    tl.collect()
    s = tl.summary()["x"]
    assert s["us"] == pytest.approx(300.0)
    # rounded as reported: GB/s to 0.1, the fraction of peak to 1e-4, elements/s to 1e-3 G
    assert s["GB/s"] == pytest.approx(8e6 / 0.3e-3 / 1e9, abs=0.05)
    assert s["frac"] == pytest.approx(8e6 / 0.3e-3 / 1e9 / bench.PEAK_GBS, abs=5e-5)
    assert s["G el/s"] == pytest.approx(2e6 / 0.3e-3 / 1e9, abs=5e-4)
    assert s["launches"] == len(ms) and np.isclose(np.median(ms), 0.3)
