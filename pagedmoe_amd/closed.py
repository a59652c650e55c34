"""Closed stitch: a decode token in one pass over the live residency table.

Reference behaviour (streaming.py:2691-2760 install and attempt, :2792-2840
arming, :2843-2870 keep-or-replay, :905-935 the per-layer closed forward):
a full stitch needs every expert in a fixed slot; this covers a model whose
experts do not all fit.  Once decode is warm (``WARM_TOKENS`` per-layer
tokens in a row fetched nothing), a decode token runs every MoE layer
against the device table as it stands -- no routed-id sync per layer -- while
a device counter adds up the routed experts the table does not hold
(``pmoe_count_missing``; a missing expert contributes a zero row).  After
the token the counter is read once.  Zero: the token is exact and kept.
Anything else: the KV cache is rewound by that token, the token runs again
through the per-layer path (which pages the misses in), and closed attempts
sit out ``COOLDOWN`` tokens.  So a stale or cold table never changes an
output; it only costs a replay.

Scope of an attempt: batch-1, one-token model calls, flow decode off (a
flow token is already one pass) and no full stitch.  A prompt, a replay or
flow disarms it; a call with a cache that cannot be rewound is never
attempted.

Rewinding.  Each layer cache of the call's ``cache`` argument (a list, or a
single cache) must drop its last token: ``trim(1)`` returning 1, mlx-lm's
KVCache interface.  ``install(model, rewind=fn)`` takes a callable
``fn(cache)`` for other cache types.

Recency.  A kept closed token makes no fetch, so it moves no expert to MRU
(as in the reference, where a closed token records only a stitch forward).
"""

from __future__ import annotations

from . import config
from ._lib import PmoeError

WARM_TOKENS = 4
COOLDOWN = 32


def _call_parts(args, kwargs):
    """(inputs, cache) of a model call ``model(inputs, cache=...)``."""
    inputs = args[0] if args else kwargs.get("inputs", kwargs.get("x"))
    cache = kwargs.get("cache")
    if cache is None and len(args) > 1:
        cache = args[1]
    return inputs, cache


def _one_token(inputs) -> bool:
    shape = getattr(inputs, "shape", None)
    return shape is not None and len(shape) >= 2 and int(shape[0]) == 1 and int(shape[1]) == 1


def _layers_of(cache):
    return list(cache) if isinstance(cache, (list, tuple)) else [cache]


def trimmable(cache) -> bool:
    return cache is not None and all(
        c is not None and callable(getattr(c, "trim", None))
        and bool(getattr(c, "is_trimmable", lambda: True)()) for c in _layers_of(cache))


def trim_one(cache) -> None:
    """Drop the last token of every layer cache (mlx-lm's trim)."""
    for c in _layers_of(cache):
        got = c.trim(1)
        if got != 1:
            raise PmoeError(f"closed stitch could not rewind a layer cache: trim(1) gave {got}")


def install(model, rewind=None) -> bool:
    """Give ``model`` (patched by patch_model) closed-stitch decode.  Bound
    to the instance: other models of the class are untouched.  False when
    ``config.STITCH`` / ``config.STITCH_PARTIAL`` is off, the model is not
    patched, or every expert is stitched already."""
    if not (config.STITCH and config.STITCH_PARTIAL):
        return False
    ring = getattr(model, "_pagedmoe_ring", None)
    cache = getattr(model, "_pagedmoe_cache", None)
    if ring is None or cache is None or cache.stitched:
        return False
    if getattr(model.__dict__.get("forward"), "closed_stitch", False):
        return True
    stock = type(model).forward.__get__(model)
    undo = rewind or trim_one
    can_undo = (lambda kv: kv is not None) if rewind is not None else trimmable

    def per_layer(args, kwargs):
        before = cache.raw_stats().misses
        out = stock(*args, **kwargs)
        if ring.closed_cooldown > 0:
            ring.closed_cooldown -= 1
            ring.warm_streak = 0
        elif cache.raw_stats().misses == before:
            ring.warm_streak += 1
            if ring.warm_streak >= WARM_TOKENS:
                ring.closed_armed = True
        else:
            ring.warm_streak = 0
        return out

    def forward(*args, **kwargs):
        inputs, kv = _call_parts(args, kwargs)
        if not _one_token(inputs) or ring.flow or cache.stitched:
            ring.closed_armed = False          # a prompt or flow: start warming again
            ring.warm_streak = 0
            return stock(*args, **kwargs)
        if not (ring.closed_armed and can_undo(kv)):
            return per_layer(args, kwargs)
        ring.begin_closed()
        try:
            out = stock(*args, **kwargs)
        finally:
            ring.closed_active = False
        if ring.end_closed() == 0:
            ring.closed_ok += 1
            return out
        ring.closed_replay += 1
        ring.closed_armed = False
        ring.warm_streak = 0
        ring.closed_cooldown = COOLDOWN
        undo(kv)
        return stock(*args, **kwargs)

    forward.closed_stitch = True
    object.__setattr__(model, "forward", forward)
    ring.closed_live = True
    return True


def uninstall(model) -> None:
    if getattr(model.__dict__.get("forward"), "closed_stitch", False):
        del model.__dict__["forward"]
        ring = getattr(model, "_pagedmoe_ring", None)
        if ring is not None:
            ring.closed_live = ring.closed_armed = False
