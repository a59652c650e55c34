"""The route-prediction governor (governor.PredictGovernor) on simulated
token timings, on the CPU: it alternates prediction on and off per window,
pairs neighbouring windows, settles on the faster state once the evidence
clears the margin and the error band, holds that decision, and is not
fooled by a steady drift in speed (reference behaviour:
streaming.py:1790-1970, measured A/B of prediction)."""

import pytest

from pagedmoe_amd import config, governor as G


class FakeRing:
    def __init__(self):
        self.predict_depth = 3


def run(gov, ring, ms_on, ms_off, tokens, monkeypatch, jitter=0.0, drift=0.0):
    """Feed ``tokens`` token boundaries whose intervals depend on the state
    the ring is in; ``drift`` adds a steady slow-down per token (ms).  The
    clock carries on across calls for one governor."""
    t = gov.__dict__.setdefault("_test_clock", [0.0])
    monkeypatch.setattr(G.time, "perf_counter", lambda: t[0])
    states = []
    for i in range(tokens):
        on = ring.predict_depth > 0
        states.append(on)
        step = (ms_on if on else ms_off) * (1.0 + jitter * ((i * 7919) % 13 - 6) / 6.0)
        t[0] += (step + drift * i) / 1e3
        gov.token()
    return states


@pytest.fixture
def knobs(monkeypatch):
    monkeypatch.setattr(config, "PREDICT_WINDOW", 8)
    monkeypatch.setattr(config, "PREDICT_MIN_TOKENS", 96)
    monkeypatch.setattr(config, "PREDICT_MARGIN", 1.03)
    monkeypatch.setattr(config, "PREDICT_Z", 2.0)
    monkeypatch.setattr(config, "PREDICT_MAX_PROBE", 6)
    monkeypatch.setattr(config, "PREDICT_HOLD", 128)


@pytest.mark.parametrize("ms_on,ms_off,want", [(6.3, 5.4, False), (4.5, 5.4, True)])
def test_governor_settles_on_the_faster_state(knobs, monkeypatch, ms_on, ms_off, want):
    ring = FakeRing()
    gov = G.PredictGovernor(ring, "auto")
    states = run(gov, ring, ms_on, ms_off, 400, monkeypatch, jitter=0.05)
    assert gov.decision is want and not gov.probing
    assert (ring.predict_depth > 0) is want
    assert any(states[:200]) and not all(states[:200])        # it did probe both
    assert all(s is want for s in states[-100:])              # and holds the decision
    assert gov.log and gov.log[-1].startswith("on" if want else "off")


def test_governor_off_when_no_measurable_difference(knobs, monkeypatch):
    monkeypatch.setattr(config, "PREDICT_MIN_TOKENS", 32)
    monkeypatch.setattr(config, "PREDICT_MAX_PROBE", 3)
    ring = FakeRing()
    gov = G.PredictGovernor(ring, "auto")
    run(gov, ring, 5.0, 5.0, 400, monkeypatch, jitter=0.3)
    assert gov.decision is False and "no measurable difference" in gov.log[-1]


def test_steady_drift_does_not_decide_for_either_state(knobs, monkeypatch):
    """Both states equally fast while every token gets slower: the pairs
    alternate which state runs first, so the trend cancels and the governor
    ends undecided-off, never "on"."""
    monkeypatch.setattr(config, "PREDICT_MIN_TOKENS", 32)
    monkeypatch.setattr(config, "PREDICT_MAX_PROBE", 4)
    ring = FakeRing()
    gov = G.PredictGovernor(ring, "auto")
    run(gov, ring, 5.0, 5.0, 600, monkeypatch, drift=0.01)
    assert gov.log and all("no measurable difference" in line for line in gov.log)


def test_idle_gaps_are_not_evidence(knobs, monkeypatch):
    """A window containing a long pause between tokens is dropped, so pauses
    that happen to fall in the on-windows do not make prediction look slow."""
    ring = FakeRing()
    gov = G.PredictGovernor(ring, "auto")
    t = [0.0]
    monkeypatch.setattr(G.time, "perf_counter", lambda: t[0])
    for i in range(800):
        on = ring.predict_depth > 0
        t[0] += (4.5e-3 if on else 5.4e-3) + (2.0 if on and i % 50 == 0 else 0.0)
        gov.token()
    assert gov.decision is True


def test_decision_is_reprobed_after_the_hold(knobs, monkeypatch):
    monkeypatch.setattr(config, "PREDICT_HOLD", 4)
    ring = FakeRing()
    gov = G.PredictGovernor(ring, "auto")
    run(gov, ring, 4.5, 5.4, 400, monkeypatch)
    assert gov.log[0].startswith("on")
    run(gov, ring, 7.0, 5.4, 1200, monkeypatch)               # prediction became costly
    assert gov.log[-1].startswith("off") and gov.decision is False


def test_pinned_modes_do_not_probe(monkeypatch):
    for mode, depth in (("on", 3), ("off", 0)):
        ring = FakeRing()
        gov = G.PredictGovernor(ring, mode)
        run(gov, ring, 9.0, 1.0, 300, monkeypatch)
        assert ring.predict_depth == depth and gov.decision is None
