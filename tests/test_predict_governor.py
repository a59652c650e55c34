"""The route-prediction A/B governor (ring.PredictGovernor) on simulated
token timings, on the CPU: it alternates prediction on and off per window,
settles on the faster state once each side has enough evidence and the gap
clears the margin and the error bar, and holds that decision
(streaming.py:1790-1970 behaviour)."""

import pytest

from pagedmoe_amd import config, ring as R


class FakeRing:
    def __init__(self):
        self.predict_depth = 3


def run(gov, ring, ms_on, ms_off, tokens, monkeypatch, jitter=0.0):
    t = [0.0]
    monkeypatch.setattr(R.time, "perf_counter", lambda: t[0])
    states = []
    for i in range(tokens):
        on = ring.predict_depth > 0
        states.append(on)
        step = (ms_on if on else ms_off) * (1.0 + jitter * ((i * 7919) % 13 - 6) / 6.0)
        t[0] += step / 1e3
        gov.token()
    return states


@pytest.mark.parametrize("ms_on,ms_off,want", [(6.3, 5.4, False), (4.5, 5.4, True)])
def test_governor_settles_on_the_faster_state(monkeypatch, ms_on, ms_off, want):
    monkeypatch.setattr(config, "PREDICT_WINDOW", 8)
    monkeypatch.setattr(config, "PREDICT_MIN_TOKENS", 96)
    ring = FakeRing()
    gov = R.PredictGovernor(ring, "auto")
    states = run(gov, ring, ms_on, ms_off, 400, monkeypatch, jitter=0.05)
    assert gov.decision is want and not gov.probing
    assert (ring.predict_depth > 0) is want
    assert any(states[:200]) and not all(states[:200])        # it did probe both
    tail = states[-100:]
    assert all(s is want for s in tail)                       # and holds the decision


def test_governor_off_when_no_measurable_difference(monkeypatch):
    monkeypatch.setattr(config, "PREDICT_WINDOW", 8)
    monkeypatch.setattr(config, "PREDICT_MIN_TOKENS", 32)
    monkeypatch.setattr(config, "PREDICT_MAX_PROBE", 3)
    ring = FakeRing()
    gov = R.PredictGovernor(ring, "auto")
    run(gov, ring, 5.0, 5.0, 400, monkeypatch, jitter=0.3)
    assert gov.decision is False and "no measurable difference" in gov.log[-1]


def test_pinned_modes_do_not_probe(monkeypatch):
    for mode, depth in (("on", 3), ("off", 0)):
        ring = FakeRing()
        gov = R.PredictGovernor(ring, mode)
        run(gov, ring, 9.0, 1.0, 300, monkeypatch)
        assert ring.predict_depth == depth and gov.decision is None
