"""Whether route prediction pays, decided from measured decode speed.

The reference measures instead of modelling (streaming.py:1790-1970): a
wrong guess costs copy bandwidth, a right one hides a miss, and which wins
depends on the link, the model and the prompt.  Mode "on" / "off" pins
prediction; "auto" runs this governor.

Paired windows.  Decode tokens are grouped into windows of
``config.PREDICT_WINDOW`` tokens, and windows alternate prediction on and
off.  Two adjacent windows (one of each state) make one sample

    d = ln(seconds per token with prediction off / with it on),

positive when prediction is faster.  Pairing neighbours cancels slow drift
in the workload (context length, routing mix, other processes) that would
bias pooled per-state means, and the pairs alternate which state runs first
(on,off | off,on | ...), so a steady trend adds to half the samples and
subtracts from the other half.  Once the pairs cover at least
``config.PREDICT_MIN_TOKENS`` tokens of each state, the weighted mean of d
is compared with the band ``max(ln PREDICT_MARGIN, PREDICT_Z * stderr)``:
above it prediction stays on, below its negative it goes off.  With no
decision after ``PREDICT_MAX_PROBE`` times that evidence, prediction goes
off (the difference is below what can be measured, and guesses still use
the link).  A decision stands for ``config.PREDICT_HOLD`` windows; then
probing resumes with the older samples' weight halved, so a changed
workload can overturn it.

A window in which any token interval exceeds ``IDLE_GAP_S`` is dropped:
it timed the caller between requests, not the decode.
"""

from __future__ import annotations

import math
import time

from . import config

IDLE_GAP_S = 1.0
MODES = ("on", "off", "auto")


class PredictGovernor:
    """Sets ``ring.predict_depth`` to its configured depth (on) or 0 (off).
    ``token()`` is called at every decode token boundary."""

    def __init__(self, ring, mode: str):
        self.ring = ring
        self.depth = ring.predict_depth
        self.mode = mode if mode in MODES else "auto"
        self.decision = None          # True / False once decided
        self.log: list = []           # one line per decision
        self._samples: list = []      # [weight, d] per pair of windows
        self._first = None            # (state, seconds per token) awaiting its partner
        self._hold = 0                # windows left before probing resumes
        self._last = None             # timestamp of the previous token
        self._n = 0                   # tokens in the current window
        self._secs = 0.0
        self._spoiled = False
        if self.mode == "off":
            ring.predict_depth = 0

    # -------------------------------------------------------------- control

    @property
    def probing(self) -> bool:
        return self.mode == "auto" and self.decision is None

    def set_mode(self, mode: str) -> None:
        self.mode = mode if mode in MODES else "auto"
        self.ring.predict_depth = 0 if self.mode == "off" else self.depth
        self.decision = None
        self._samples.clear()
        self._first = None
        self._restart_window()

    def describe(self) -> dict:
        return {"mode": self.mode, "decision": self.decision, "probing": self.probing,
                "depth": self.ring.predict_depth, "pairs": len(self._samples),
                "mean_log_ratio": self._mean_var()[0] if self._samples else None}

    # -------------------------------------------------------------- measurement

    def token(self) -> None:
        if self.mode != "auto" or self.depth <= 0:
            return
        now = time.perf_counter()
        last, self._last = self._last, now
        if last is None:
            return
        gap = now - last
        if gap > IDLE_GAP_S:
            self._spoiled = True
        self._n += 1
        self._secs += gap
        if self._n >= max(2, int(config.PREDICT_WINDOW)):
            state, spt, ok = self.ring.predict_depth > 0, self._secs / self._n, not self._spoiled
            self._restart_window()
            if ok:
                self._window_done(state, spt)

    def _restart_window(self) -> None:
        self._n, self._secs, self._spoiled = 0, 0.0, False

    def _set(self, on: bool) -> None:
        self.ring.predict_depth = self.depth if on else 0

    def _window_done(self, state: bool, spt: float) -> None:
        if self.decision is not None:
            self._hold -= 1
            if self._hold <= 0:               # probe again, older evidence discounted
                for s in self._samples:
                    s[0] *= 0.5
                self.decision = None
                self._first = None
                self._set(True)
            return
        if self._first is None or self._first[0] == state:
            self._first = (state, spt)
            self._set(not state)              # the partner window runs the other state
            return
        on_spt, off_spt = (spt, self._first[1]) if state else (self._first[1], spt)
        self._first = None
        self._samples.append([1.0, math.log(off_spt / on_spt)])
        # the next pair opens with the state that just ran (on,off | off,on
        # | on,off ...), so a steady drift in speed favours neither state
        self._set(state)
        self._judge()

    def _mean_var(self):
        w = sum(s[0] for s in self._samples)
        mean = sum(s[0] * s[1] for s in self._samples) / w
        if w <= 1.0:
            return mean, math.inf, w
        var = sum(s[0] * (s[1] - mean) ** 2 for s in self._samples) / (w - 1.0)
        return mean, var, w

    def _judge(self) -> None:
        mean, var, w = self._mean_var()
        per_side = w * max(2, int(config.PREDICT_WINDOW))
        need = max(int(config.PREDICT_MIN_TOKENS), int(config.PREDICT_WINDOW))
        if per_side < need or len(self._samples) < 2:
            return
        stderr = math.sqrt(var / w)
        band = max(math.log(float(config.PREDICT_MARGIN)), float(config.PREDICT_Z) * stderr)
        gain = math.exp(mean) - 1.0
        what = (f"prediction {100 * gain:+.1f}% tokens/s over {len(self._samples)} window "
                f"pairs (band +/-{100 * (math.exp(band) - 1):.1f}%)")
        if mean > band:
            self._decide(True, "on: " + what)
        elif mean < -band:
            self._decide(False, "off: " + what)
        elif per_side >= need * max(1, int(config.PREDICT_MAX_PROBE)):
            self._decide(False, "off, no measurable difference: " + what)

    def _decide(self, on: bool, why: str) -> None:
        self.decision = on
        self._hold = max(1, int(config.PREDICT_HOLD))
        self._set(on)
        self.log.append(why)
