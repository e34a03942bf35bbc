"""bench.py's host-side pieces on the CPU: the multi-GPU refusal, the per-replay statistics, the
strict workspace bound, and the clock warm-up's replay accounting (it must keep the timed replays
aligned with the start of the graph cycle)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_replay_stats_per_step():
    st = bench.replay_stats([4.0, 8.0, 6.0], 4)
    assert st["replays"] == 3 and st["steps_per_replay"] == 4
    assert st["median_ms"] == 1.5 and st["min_ms"] == 1.0 and st["max_ms"] == 2.0
    assert st["mean_ms"] == pytest.approx(1.5)


def test_strict_rows_for_mode_and_bound():
    assert bench.strict_rows_for("strict", 1) == 1
    assert bench.strict_rows_for("strict", 16) == 16
    assert bench.strict_rows_for("fast", 16) == 0
    assert bench.strict_rows_for("strict", 512) == 0        # beyond 64 rows / 256 slots: fast geometry


class _FakeCuda:
    def __init__(self):
        self.syncs = 0

    def synchronize(self):
        self.syncs += 1

    def stream(self, s):
        class _Ctx:
            def __enter__(self):
                return s

            def __exit__(self, *a):
                return False
        return _Ctx()


class _FakeTorch:
    def __init__(self):
        self.cuda = _FakeCuda()


@pytest.mark.parametrize("unit", [1, 2, 8])
def test_clock_warmup_replays_whole_cycles(unit):
    torch = _FakeTorch()
    calls = []
    n, ms = bench.clock_warmup(torch, None, lambda: calls.append(1), 5.0, unit)
    assert n == len(calls) and n > 0 and n % unit == 0        # the cycle position is unchanged
    assert ms >= 5.0 and torch.cuda.syncs >= 1
    assert bench.clock_warmup(torch, None, lambda: calls.append(1), 0.0, unit) == (0, 0.0)
