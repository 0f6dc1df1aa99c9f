"""The committed counter summary that bench.py's roofline.traffic reads: it parses, and the
scaled bytes per gate+up launch agree with the algorithmic bytes (2 x 12288 x 4096 packed
K=3 words), so the figure can neither vanish (a key renamed) nor drift below the bytes the
kernel must read (a wrong calibration pass). Also bench.py's host logic that needs no GPU:
it refuses more than one GPU, and its timed region holds exactly the requested blocks."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

ALGORITHMIC = 2 * 12288 * 4096 * 3 // 8


def test_traffic_profile_parses_and_covers_the_packed_bytes():
    t = bench.traffic_from_profile()
    assert t is not None, "profiles/gemv_gate_up_b1_traffic.txt missing a key bench.py reads"
    # every packed word once, plus activations, scales and fold inputs: a few percent more
    assert 1.0 <= t / ALGORITHMIC <= 1.1, t / ALGORITHMIC


def test_dram_counters_agree_with_the_scaled_fetch():
    vals = {}
    for line in open(bench.TRAFFIC_FILE):
        parts = line.split()
        if len(parts) == 2 and not line.startswith("#"):
            vals[parts[0]] = float(parts[1])
    # the DRAM request counters need no scale (the 1 GiB calibration sum reads 1 GiB by them)
    assert abs(vals["cal_read_dram_kib"] / vals["cal_kib"] - 1.0) < 0.01
    dram = vals["dram_read_kib"] * 1024
    assert 1.0 <= dram / ALGORITHMIC <= 1.1
    scaled = vals["fetch_kib"] * vals["cal_kib"] / vals["cal_read_fetch_kib"] * 1024
    assert abs(scaled / dram - 1.0) < 0.05


def test_traffic_absent_file_is_none(tmp_path):
    assert bench.traffic_from_profile(str(tmp_path / "missing.txt")) is None


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with a message (one GPU is what this build measures),
    before it touches the GPU."""
    import json
    import subprocess
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_time_blocks_times_exactly_the_steps(monkeypatch):
    """The timed region of the block bench holds exactly `steps` blocks, block i on weight
    copy i % copies, whatever `steps` is against the run length (whole runs, then a tail)."""
    import types
    log = []

    class Graph:
        def __init__(self, fn):
            self.fn = fn

        def replay(self):
            self.fn()

    monkeypatch.setattr(bench, "capture", lambda torch, fn: Graph(fn))
    fake = types.SimpleNamespace(cuda=types.SimpleNamespace(synchronize=lambda: log.append("sync")))
    for copies, steps, warmup in [(14, 200, 10), (14, 28, 3), (5, 3, 0), (18, 200, 20), (1, 7, 2)]:
        log.clear()
        sec = bench.time_blocks(fake, lambda c: log.append(c), copies, steps, warmup)
        assert sec >= 0
        syncs = [i for i, v in enumerate(log) if v == "sync"]
        timed = log[syncs[-2] + 1:syncs[-1]]               # between the last two syncs
        assert timed == [i % copies for i in range(steps)], (copies, steps)
        warm = [v for v in log[:syncs[-2]] if v != "sync"]
        assert len(warm) >= max(warmup, 1) and len(warm) % copies == 0   # whole runs


def test_warm_up_lasts_the_count_and_the_time(monkeypatch):
    import time
    import types
    monkeypatch.setattr(bench, "WARM_S", 0.02)
    calls = []
    fake = types.SimpleNamespace(cuda=types.SimpleNamespace(synchronize=lambda: None))
    t0 = time.perf_counter()
    n = bench.warm_up(fake, lambda i: calls.append(i), 3)
    assert time.perf_counter() - t0 >= 0.02 and n == len(calls) >= 3
    assert calls == list(range(n))
    calls.clear()
    monkeypatch.setattr(bench, "WARM_S", 0.0)
    assert bench.warm_up(fake, lambda i: calls.append(i), 5) == 5 and calls == list(range(5))
