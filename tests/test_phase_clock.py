"""The profile-mode phase clock of the host decode loops (reference spec.py:112-121, 133-149): it
accumulates each phase's wall time and marks every phase as one roctx range, pushed and popped in
order and never left open across steps; the decode-loop clock brackets a loop with one range when
stats are asked for. Runs on the CPU (the device synchronisation and the range calls are recorded
instead of made)."""

import torch

from skinny_mlx import spec


def _record(monkeypatch):
    calls = []
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda name: calls.append(("push", name)))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: calls.append(("pop", None)))
    return calls


def test_phase_clock_ranges_follow_the_phases(monkeypatch):
    calls = _record(monkeypatch)
    clock = spec._PhaseClock(True)
    for _ in range(2):
        clock.start()
        for phase in spec._PhaseClock.PHASES:
            clock.lap(phase)
    names = [n for kind, n in calls if kind == "push"]
    assert names == [f"skinny:{p}" for p in spec._PhaseClock.PHASES] * 2
    depth = 0
    for kind, _ in calls:
        depth += 1 if kind == "push" else -1
        assert depth in (0, 1)
    assert depth == 0 and not clock.open
    assert set(clock.total) == set(spec._PhaseClock.PHASES) and all(v >= 0 for v in clock.total.values())


def test_phase_clock_off_makes_no_calls(monkeypatch):
    calls = _record(monkeypatch)
    clock = spec._PhaseClock(False)
    clock.start()
    clock.lap("draft")
    assert calls == [] and all(v == 0 for v in clock.total.values())


def test_a_step_cut_short_closes_its_range_at_the_next_start(monkeypatch):
    calls = _record(monkeypatch)
    clock = spec._PhaseClock(True)
    clock.start()
    clock.lap("draft")  # the step ends early (the loop's last step)
    clock.start()
    depth = 0
    for kind, _ in calls:
        depth += 1 if kind == "push" else -1
        assert depth in (0, 1)
    assert depth == 1 and clock.open


def test_loop_clock_brackets_the_loop_only_with_stats(monkeypatch):
    calls = _record(monkeypatch)
    st = {}
    clock = spec._LoopClock(st)
    clock.start()
    clock.stop(10)
    assert calls == [("push", "skinny:decode_loop"), ("pop", None)]
    assert st["decode_tok_s"] >= 0 and "decode_ms" in st
    calls.clear()
    quiet = spec._LoopClock(None)
    quiet.start()
    quiet.stop(10)
    assert calls == []
