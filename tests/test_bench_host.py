"""bench.py's host logic on the CPU: the one-GPU rule, the clock settling
loop and the traffic figure's tie to the profiled code object. No device."""
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


class FakeDev:
    """HIP events that report a scripted duration for each batch."""

    def __init__(self, batch_ms):
        self.batch_ms = list(batch_ms)
        self.done = 0
        self.launches = 0

    def events(self, n):
        assert n == 2

    def record(self, i):
        pass

    def sync(self):
        pass

    def elapsed(self, a, b):
        ms = self.batch_ms[min(self.done, len(self.batch_ms) - 1)]
        self.done += 1
        return ms


def launches_of(dev):
    def launch():
        dev.launches += 1
    return launch


def test_settle_runs_through_the_ramp_and_stops_when_steady(bench):
    # per-launch us of each batch of 25: idle clocks, the ramp, then steady
    us = [65.0, 69.2, 76.5, 74.6, 71.3, 67.8, 66.1, 65.0, 64.3, 64.1, 64.1, 64.0, 64.1, 64.1]
    dev = FakeDev([u * 25 / 1e3 for u in us])
    st = bench.settle(dev, launches_of(dev), batch=25, min_ms=0.0)
    # 64.3 -> 64.1 -> 64.1 -> 64.0 is the first run of three calm batches
    assert st["launches"] == 25 * 12 == dev.launches
    assert st["first_batch_us"] == 65.0 and st["max_batch_us"] == 76.5 and st["last_batch_us"] == 64.0


def test_settle_keeps_going_until_the_minimum_time(bench):
    dev = FakeDev([64.0 * 25 / 1e3] * 100)          # steady from the start, 1.6 ms per batch
    st = bench.settle(dev, launches_of(dev), batch=25, min_ms=25.0)
    assert st["launches"] == 25 * 16                 # 16 batches reach 25.6 ms


def test_settle_gives_up_after_max_batches(bench):
    dev = FakeDev([(60.0 + 5.0 * (i % 2)) * 25 / 1e3 for i in range(200)])   # never steady
    st = bench.settle(dev, launches_of(dev), batch=25, max_batches=80)
    assert st["launches"] == 25 * 80


def test_traffic_is_reported_only_for_the_profiled_code_object(bench, tmp_path, monkeypatch):
    prof = tmp_path / "traffic.json"
    prof.write_text(json.dumps({"hbm_bytes_per_launch": 430000000, "code_object_sha256": "ab" * 32}))
    monkeypatch.setattr(bench, "TRAFFIC_JSON", str(prof))
    monkeypatch.setattr(bench, "code_object_sha256", lambda: "ab" * 32)
    assert bench.profiled_traffic()[0] == 430000000
    monkeypatch.setattr(bench, "code_object_sha256", lambda: "cd" * 32)
    value, why = bench.profiled_traffic()
    assert value is None and "another build" in why
    monkeypatch.setattr(bench, "code_object_sha256", lambda: None)
    assert bench.profiled_traffic()[0] is None
    monkeypatch.setattr(bench, "TRAFFIC_JSON", str(tmp_path / "missing.json"))
    assert bench.profiled_traffic() == (None, "no traffic profile")


def test_committed_traffic_profile_matches_the_committed_build(bench):
    """The committed profile names the code object it was taken on; when the
    tree holds that build, the bench reports its figure."""
    with open(bench.TRAFFIC_JSON) as f:
        t = json.load(f)
    assert t["kernel"] == "sllm_k_gemv_slab" and len(t["code_object_sha256"]) == 64
    assert 1.0 <= t["ratio"] < 1.05
    cur = bench.code_object_sha256()
    if cur is not None and cur == t["code_object_sha256"]:
        assert bench.profiled_traffic()[0] == t["hbm_bytes_per_launch"]
