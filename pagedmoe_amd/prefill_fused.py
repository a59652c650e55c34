"""One MoE pass per prompt chunk: decoder layers that split only their attention.

Behaviour of the reference's fused prefill (prefill_fused.py:1-43 for the
idea, :195-245 and :248-307 for the two layer shapes, :335-411 for install):
a long prompt chunk routes to nearly every expert of every layer, so a
prefill streams the expert mass once per MoE call of a layer.  Attention's
score matrix is what bounds how many rows one call can take; the MoE has no
such bound.  So inside one decoder layer attention runs over row splits
sized for the score budget, each split appending its keys to the layer's KV
cache exactly as consecutive model calls would, and the feed-forward block
runs once over every row.  Each token sees the same attention arithmetic on
the same inputs; only the number of expert passes changes.

How it is put together here:

* Per instance, never per class.  ``install`` binds a forward to each
  eligible decoder-layer *instance*; an instance attribute shadows the
  class's method when ``nn.Module.__call__`` looks up ``forward``.  Hybrid
  stacks (Qwen3-Next) build linear-attention and full-attention layers from
  one class: a linear-attention instance, or one without ``self_attn`` or a
  feed-forward block, is simply never bound, so it keeps the stock call (a
  recurrent layer must see its whole sequence, and it has no score matrix
  to bound).  ``uninstall`` removes the instance attributes.
* Row splits from a closed form.  ``c`` query rows against ``kv`` cached
  keys materialise ``heads * c * (kv + c)`` fp32 scores; the largest ``c``
  within ``config.ATTN_SCORE_MB`` is the positive root of
  ``c^2 + kv*c - budget / (4 * heads)``, floored and clamped to
  ``[1, config.ATTN_SUB_CHUNK]``.  The keys grow split by split, so later
  splits are never larger.
* The residual stream is filled split by split.  ``h`` is allocated at the
  first split (with the dtype ``x + attn`` promotes to) and each split
  writes its rows, so no list of split outputs is held while the next
  split's scores exist.
* Two layer shapes.  Pre-norm residual blocks (Qwen3-MoE, Qwen3-Next,
  DeepSeek-V3, Kimi-K2, MiniMax: ``input_layernorm``, ``self_attn``,
  ``post_attention_layernorm`` and ``mlp`` or ``block_sparse_moe``, called
  as ``layer(x, mask, cache)``), and hyper-connection blocks
  (``attn_hyper_connection`` / ``mlp_hyper_connection`` around
  ``self_attn`` and ``mlp``, called positionally as
  ``layer(h, rope, mask, conv_mask, cache, idx_cache, ids, prev_ctx)``).

Calls of at most ``SMALL_CALL_ROWS`` rows (decode, speculative verify) and
calls with extra keyword arguments take the stock forward untouched.
"""

from __future__ import annotations

import math
import weakref
from typing import Any

import torch

from . import config

SMALL_CALL_ROWS = 8
_FFN_NAMES = ("mlp", "block_sparse_moe")
_HEAD_NAMES = ("n_heads", "num_heads", "num_attention_heads", "heads")
_bound: "weakref.WeakSet" = weakref.WeakSet()      # instances carrying a split forward


# ---------------------------------------------------------------- layer shape

def feed_forward(layer: Any):
    """The instance's feed-forward module (``mlp`` or ``block_sparse_moe``),
    or None.  Per instance: some models put dense and MoE blocks under one
    class."""
    for name in _FFN_NAMES:
        mod = getattr(layer, name, None)
        if mod is not None:
            return mod
    return None


def is_linear_attention(layer: Any) -> bool:
    """A recurrent / linear-attention layer (Qwen3-Next's Gated DeltaNet
    layers and their kin), by the markers hybrid models set on it."""
    if getattr(layer, "layer_type", None) == "linear_attention":
        return True
    if getattr(layer, "is_linear", False):
        return True
    return hasattr(layer, "linear_attn") and not hasattr(layer, "self_attn")


def layer_shape(layer: Any) -> str | None:
    """"hyper", "pre_norm", or None when this instance must keep its stock
    call (no full attention to split, or no feed-forward block)."""
    if is_linear_attention(layer) or not hasattr(layer, "self_attn"):
        return None
    if feed_forward(layer) is None:
        return None
    if hasattr(layer, "attn_hyper_connection") and hasattr(layer, "mlp_hyper_connection"):
        return "hyper"
    if hasattr(layer, "input_layernorm") and hasattr(layer, "post_attention_layernorm"):
        return "pre_norm"
    return None


def layer_is_fusable(layer: Any) -> bool:
    return layer_shape(layer) is not None


# ---------------------------------------------------------------- row splits

def attention_heads(layer: Any) -> int:
    attn = getattr(layer, "self_attn", None)
    for name in _HEAD_NAMES:
        v = getattr(attn, name, None)
        if isinstance(v, int) and v > 0:
            return v
    return 1


def rows_for_budget(heads: int, kv: int, budget_bytes: int, cap: int) -> int:
    """Largest c in [1, cap] with 4 * heads * c * (kv + c) <= budget_bytes."""
    q = budget_bytes // (4 * max(1, heads))             # score pairs allowed
    c = (math.isqrt(kv * kv + 4 * q) - kv) // 2          # floor of the positive root
    c = max(1, min(int(cap), c))
    while c > 1 and c * (kv + c) > q:                    # isqrt rounding, either way
        c -= 1
    while c < cap and (c + 1) * (kv + c + 1) <= q:
        c += 1
    return c


def row_splits(layer: Any, total: int, kv0: int) -> list:
    """[(start, end)] covering [0, total): each split sized for the keys
    cached when it runs (kv0 before the call, plus the earlier splits)."""
    heads = attention_heads(layer)
    budget = max(1, int(config.ATTN_SCORE_MB)) << 20
    cap = max(1, int(config.ATTN_SUB_CHUNK))
    out, start = [], 0
    while start < total:
        end = min(total, start + rows_for_budget(heads, kv0 + start, budget, cap))
        out.append((start, end))
        start = end
    return out



def cached_keys(cache: Any) -> int:
    """Keys one layer's cache already holds (its ``offset``; a layer that
    keeps a list of caches reports the first).  0 without a cache."""
    if isinstance(cache, (list, tuple)):
        cache = cache[0] if cache else None
    if cache is None:
        return 0
    off = getattr(cache, "offset", 0)
    try:
        return max(0, int(off))
    except (TypeError, ValueError):
        return 0


def mask_rows(mask: Any, start: int, end: int, keys: int):
    """The rows of the chunk's mask for split [start, end) against the first
    ``keys`` keys.  None and string masks ("causal") pass through: they align
    queries to the end of the keys by themselves."""
    if mask is None or isinstance(mask, str):
        return mask
    return mask[..., start:end, :keys]


# ---------------------------------------------------------------- forwards

def _stock(layer):
    return type(layer).forward.__get__(layer)


def _pre_norm_forward(layer):
    stock = _stock(layer)

    def forward(x, mask=None, cache=None, **kw):
        if kw or x.dim() != 3 or x.shape[1] <= SMALL_CALL_ROWS:
            return stock(x, mask, cache, **kw)
        total = int(x.shape[1])
        kv0 = cached_keys(cache)
        splits = row_splits(layer, total, kv0)
        if len(splits) == 1:
            return stock(x, mask, cache)
        h = None
        for start, end in splits:
            r = layer.self_attn(layer.input_layernorm(x[:, start:end]),
                                mask_rows(mask, start, end, kv0 + end), cache)
            if h is None:
                h = torch.empty(x.shape[:-1] + r.shape[-1:], dtype=torch.result_type(x, r),
                                device=x.device)
            h[:, start:end] = x[:, start:end] + r
            del r
        return h + feed_forward(layer)(layer.post_attention_layernorm(h))

    return forward


def _hyper_forward(layer):
    stock = _stock(layer)

    def forward(h, rope=None, mask=None, conv_mask=None, cache=None, idx_cache=None, ids=None,
                prev_ctx=None, *args, **kw):
        def plain():
            return stock(h, rope, mask, conv_mask, cache, idx_cache, ids, prev_ctx, *args, **kw)

        if args or kw or h is None or h.dim() != 3 or h.shape[1] <= SMALL_CALL_ROWS:
            return plain()
        total = int(h.shape[1])
        kv0 = cached_keys(cache)
        splits = row_splits(layer, total, kv0)
        if len(splits) == 1:
            return plain()
        ple = getattr(layer, "ple", None)
        if ple is not None:
            h = h + ple(h, ids, prev_ctx, cache)
        x, carry, inject = layer.attn_hyper_connection(h)
        att = None
        for start, end in splits:
            r = layer.self_attn(x[:, start:end], rope, mask_rows(mask, start, end, kv0 + end),
                                cache, idx_cache)
            if att is None:
                att = torch.empty(x.shape[:-1] + r.shape[-1:], dtype=r.dtype, device=r.device)
            att[:, start:end] = r
            del r
        h = carry + (att.unsqueeze(-2) * inject.unsqueeze(-1)).flatten(-2)
        x, carry, inject = layer.mlp_hyper_connection(h)
        y = layer.mlp(x)
        return carry + (y.unsqueeze(-2) * inject.unsqueeze(-1)).flatten(-2)

    return forward


_MAKERS = {"pre_norm": _pre_norm_forward, "hyper": _hyper_forward}


# ---------------------------------------------------------------- install

def decoder_layers(model: Any):
    """The decoder layer list of a model: model.model.layers,
    model.language_model.model.layers or model.layers."""
    for path in (("model", "layers"), ("language_model", "model", "layers"), ("layers",)):
        obj = model
        for name in path:
            obj = getattr(obj, name, None)
            if obj is None:
                break
        if obj is not None and len(obj):
            return obj
    return None


def install(model: Any) -> bool:
    """Bind the split forward to every eligible decoder-layer instance of
    ``model``.  Idempotent.  False when ``config.FUSED_PREFILL`` is off or no
    instance is eligible."""
    if not config.FUSED_PREFILL:
        return False
    layers = decoder_layers(model)
    if layers is None:
        return False
    n = 0
    for layer in layers:
        if layer in _bound:
            n += 1
            continue
        shape = layer_shape(layer)
        if shape is None:
            continue
        fwd = _MAKERS[shape](layer)
        fwd.split_shape = shape
        object.__setattr__(layer, "forward", fwd)
        _bound.add(layer)
        n += 1
    return n > 0


def installed(layer: Any) -> bool:
    return layer in _bound


def uninstall(model: Any = None) -> None:
    """Remove the split forward from the instances of ``model`` (every
    bound instance without one)."""
    layers = list(_bound) if model is None else list(decoder_layers(model) or [])
    for layer in layers:
        if layer in _bound:
            layer.__dict__.pop("forward", None)
            _bound.discard(layer)
