"""The tuner's confirmation round on the CPU (the GPU timer replaced by a
stand-in): only candidates near the fastest first-pass time are re-timed,
in turn, and the winner is the lowest median, so a first-pass timing that
drifted low does not decide alone."""
from aiter_amd import tuner


def test_confirm_takes_lowest_median(monkeypatch):
    # later timings of each candidate by name; "a" was lucky in the first pass
    later = {"a": [1.20, 1.25], "b": [1.05, 1.06], "c": [1.30, 1.31], "far": [0.5, 0.5]}
    calls = []

    def fake_time(run, n_copies, iters):
        calls.append(run)
        return later[run].pop(0)

    monkeypatch.setattr(tuner, "time_rotated", fake_time)
    timed = [(1.00, "a", "A"), (1.07, "b", "B"), (1.02, "c", "C"), (1.50, "far", "FAR")]
    t, payload = tuner.confirm(timed, 1, 1)
    assert payload == "B" and t == 1.06
    # "far" (50% slower in the first pass) is never re-timed; the rest in turn
    assert calls == ["a", "c", "b", "a", "c", "b"]


def test_confirm_single_candidate_not_retimed(monkeypatch):
    monkeypatch.setattr(tuner, "time_rotated", lambda *a: (_ for _ in ()).throw(AssertionError("re-timed")))
    assert tuner.confirm([(2.0, "x", "X"), (3.0, "y", "Y")], 1, 1) == (2.0, "X")
