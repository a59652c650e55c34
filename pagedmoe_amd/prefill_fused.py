"""Layer-fused prefill: attention in sub-chunks, the MoE once per prompt chunk.

Counterpart of the reference's prefill_fused.py (:1-43 for the idea, install
:339-395, the patched layer call :195-245).  A long prompt chunk routes to
nearly every expert of every layer, so each model call over a chunk streams
the whole expert mass once; chunking the *model* call to bound attention's
score matrix would stream it once per chunk.  Only attention needs the small
chunk, so inside one pre-norm decoder layer:

    for each attention sub-chunk i:  r_i = self_attn(input_layernorm(x_i), mask_i, cache)
    h = x + concat(r_i)
    return h + mlp(post_attention_layernorm(h))      # once, over every token

Consecutive sub-chunks see the KV cache grow exactly as consecutive model
calls would (each appends its keys before the next runs), and sub-chunk i's
mask is rows [start, end) of the chunk's mask restricted to the keys present
after it, so each token's attention is the same arithmetic on the same
inputs.  Only the number of times the experts are streamed changes.

The layer interface is the reference's (mlx-lm's): ``layer(x, mask=None,
cache=None)`` with x [B, T, D] and submodules ``self_attn``,
``input_layernorm``, ``post_attention_layernorm`` and ``mlp`` (or
``block_sparse_moe``).  ``cache.offset`` is the number of keys already held.
Sub-chunk size: at most ``config.ATTN_SUB_CHUNK`` rows, and small enough that
heads x rows x keys fp32 scores fit ``config.ATTN_SCORE_MB`` -- the
materialised score matrix is what bounds the chunk (adaptive_prefill.py:249).
"""

from __future__ import annotations

from typing import Any

import torch

from . import config

_installed: dict = {}           # class -> original forward
_MIN_SPLIT_TOKENS = 8           # decode and verify batches take the stock call


def _ffn(layer: Any):
    for name in ("mlp", "block_sparse_moe"):
        ffn = getattr(layer, name, None)
        if ffn is not None:
            return ffn
    return None


def layer_is_fusable(layer: Any) -> bool:
    """A pre-norm decoder layer with attention and a feed-forward block."""
    return (all(hasattr(layer, a) for a in ("self_attn", "input_layernorm",
                                            "post_attention_layernorm"))
            and _ffn(layer) is not None)


def cache_offset(cache: Any) -> int:
    """Keys already in one layer's cache (0 without a cache)."""
    if cache is None:
        return 0
    off = getattr(cache, "offset", None)
    if off is None:
        try:
            off = getattr(cache[0], "offset", None)
        except (TypeError, IndexError, AttributeError, KeyError):
            off = None
    try:
        return max(0, int(off))
    except (TypeError, ValueError):
        return 0


def _heads(layer: Any) -> int:
    attn = getattr(layer, "self_attn", None)
    for name in ("n_heads", "num_heads", "num_attention_heads", "heads"):
        v = getattr(attn, name, None)
        if isinstance(v, int) and v > 0:
            return v
    return 1


def attention_sub_chunk(layer: Any, kv_len: int) -> int:
    """Query rows one attention call may take against kv_len keys already
    cached: the largest C <= ATTN_SUB_CHUNK with
    heads * C * (kv_len + C) * 4 <= ATTN_SCORE_MB, and at least 1."""
    cap = max(1, int(config.ATTN_SUB_CHUNK))
    budget = max(1, int(config.ATTN_SCORE_MB)) << 20
    per_row = 4 * _heads(layer)
    lo, hi = 1, cap
    while lo < hi:                          # largest C with the scores in budget
        mid = (lo + hi + 1) // 2
        if per_row * mid * (kv_len + mid) <= budget:
            lo = mid
        else:
            hi = mid - 1
    return lo


def attention_plan(layer: Any, total: int, offset: int) -> list:
    """[(start, end)] sub-chunks covering [0, total); each sized for the keys
    present when it runs, so later sub-chunks (longer KV) may be shorter."""
    plan, start = [], 0
    while start < total:
        n = min(attention_sub_chunk(layer, offset + start), total - start)
        plan.append((start, start + n))
        start += n
    return plan


def slice_mask(mask: Any, start: int, end: int, keys: int):
    """Rows [start, end) of the chunk's mask, keys [0, keys).  A string mask
    ("causal") aligns queries to the end of the keys by itself."""
    if mask is None or isinstance(mask, str):
        return mask
    return mask[..., start:end, :keys]


def _fused_forward(orig):
    def forward(self, x, mask=None, cache=None, **kw):
        if kw or x.dim() != 3 or x.shape[1] <= _MIN_SPLIT_TOKENS:
            return orig(self, x, mask, cache, **kw)
        ffn = _ffn(self)
        total = int(x.shape[1])
        offset = cache_offset(cache)
        plan = attention_plan(self, total, offset)
        if len(plan) <= 1:
            return orig(self, x, mask, cache)
        parts = [self.self_attn(self.input_layernorm(x[:, s:e]),
                                slice_mask(mask, s, e, offset + e), cache) for s, e in plan]
        h = x + torch.cat(parts, dim=1)
        del parts
        return h + ffn(self.post_attention_layernorm(h))

    forward.__wrapped__ = orig
    return forward


def decoder_layers(model: Any):
    """The decoder layer list of a model (model.model.layers, model.layers,
    model.language_model.model.layers)."""
    for get in (lambda m: m.model.layers, lambda m: m.layers,
                lambda m: m.language_model.model.layers):
        try:
            layers = get(model)
        except AttributeError:
            continue
        if layers is not None and len(layers):
            return layers
    return None


def install(model: Any) -> bool:
    """Patch the model's decoder layer classes so a long call sub-chunks its
    own attention and runs the MoE once.  Idempotent; False when nothing is
    fusable or config.FUSED_PREFILL is off."""
    if not config.FUSED_PREFILL:
        return False
    layers = decoder_layers(model)
    if not layers:
        return False
    patched = 0
    for layer in layers:
        cls = type(layer)
        if cls in _installed:
            patched += 1
            continue
        if not layer_is_fusable(layer):
            continue
        _installed[cls] = cls.forward
        cls.forward = _fused_forward(cls.forward)
        patched += 1
    return patched > 0


def uninstall() -> None:
    """Restore every patched class's forward."""
    for cls, orig in list(_installed.items()):
        cls.forward = orig
        del _installed[cls]
