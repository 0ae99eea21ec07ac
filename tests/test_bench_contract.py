"""bench.py's timing loop on the CPU, with a stand-in device module: a timed launch whose look-back
gave up a wait (unp_hip_exec_check reports Stalled) stops the run before any line is printed, and a
clean run reports each case's average kernel time from its event pairs."""
from __future__ import annotations

import pytest

import bench


class _Err(Exception):
    def __init__(self, kind):
        super().__init__(kind)
        self.kind = kind


class _Event:
    def elapsed_ms(self, other):
        return 0.5


class _Exec:
    def __init__(self, stalled):
        self.stalled, self.timing = stalled, []

    def set_timing(self, a, b):
        self.timing.append((a, b))

    def check(self):
        if self.stalled:
            raise _Err("Stalled")

    def last_launch(self):
        return {"entry": "k_v", "grid": [512, 1, 1]}


class _Case:
    def __init__(self, name, stalled=False):
        self.name, self.what, self.exec = name, "a case", _Exec(stalled)
        self.nbytes, self.elements, self.ops, self.launches = 4_000_000, 1_000_000, 0, 0

    def launch(self):
        self.launches += 1


class _U:
    UnpError = _Err
    Event = _Event

    @staticmethod
    def synchronize():
        pass


def test_a_stalled_launch_stops_the_bench_before_any_line():
    cases = [_Case("ok"), _Case("stalls", stalled=True)]
    with pytest.raises(SystemExit) as e:
        bench.time_cases(_U, cases, steps=3)
    assert "stalls" in str(e.value) and "Stalled" in str(e.value) and "no line is printed" in str(e.value)
    assert cases[1].launches == 3


def test_a_clean_run_reports_every_case_and_clears_the_timing():
    cases = [_Case("a"), _Case("b")]
    per = bench.time_cases(_U, cases, steps=4)
    assert [p["name"] for p in per] == ["a", "b"]
    assert all(p["us"] == 500.0 and p["entry"] == "k_v" for p in per)
    assert all(c.exec.timing[-1] == (None, None) and c.launches == 4 for c in cases)
