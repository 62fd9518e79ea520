"""bench.py's own logic on the CPU: the refusal of more than one GPU, and the settling run that every compute figure
waits for (untimed steps in groups until the time per step stops drifting: a group within 1% of the one before,
after at least min_ms, at most max_ms). The GPU timer is replaced by a stand-in that reports a given time per step
for each timed group."""
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


class FakeTimer:
    """The part of we.Graph that bench.time_launches uses; timed group i takes per_step_ms[i] per step."""

    def __init__(self, per_step_ms):
        self.per_step_ms = list(per_step_ms)
        self.groups = 0
        self.launched = 0
        self.start = 0

    def sync(self):
        pass

    def timer_start(self):
        self.start = self.launched

    def timer_stop(self):
        per = self.per_step_ms[min(self.groups, len(self.per_step_ms) - 1)]
        self.groups += 1
        return per * (self.launched - self.start)


def settle(per_step_ms, **kw):
    g = FakeTimer(per_step_ms)
    seen = []

    def step(i):
        g.launched += 1
        seen.append(i)

    res = bench.settle_steps(g, step, **kw)
    assert seen == list(range(res["steps"]))  # every step index once, in order
    return res


def test_stops_once_two_groups_agree():
    # a start transient: 1.5 ms per step falling to 0.5, then flat; the 6th group is the first within 1% of the 5th
    res = settle([1.5, 1.2, 0.9, 0.6, 0.5, 0.5, 0.5], group=10, min_ms=1.0, max_ms=1000.0)
    assert res["steps"] == 60
    assert res["first_group_us_per_step"] == 1500.0 and res["last_group_us_per_step"] == 500.0
    assert res["ms"] == pytest.approx(15 + 12 + 9 + 6 + 5 + 5)


def test_runs_at_least_min_ms():
    # 5 ms per group, flat from the start: agreement alone does not stop it before 40 ms
    assert settle([0.5] * 100, group=10, min_ms=40.0, max_ms=1000.0)["steps"] == 80


def test_gives_up_at_max_ms():
    # never within 1%: 10, 20, 10, 20, ... ms per group; the 7th group brings the total to 100 ms
    res = settle([1.0, 2.0] * 50, group=10, min_ms=0.0, max_ms=100.0)
    assert res["steps"] == 70 and res["ms"] == pytest.approx(100.0)


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert p.returncode == 2, p.stderr
    assert "one GPU" in p.stderr and not p.stdout.strip()
