"""Hot-path knobs, read from the environment once at import.

Names and defaults follow the reference's PAGED_MOE_* knobs that touch this
path (config.py): SLAB_RESERVE_FRAC :718, LFRU / LFRU_SCAN :1477-1478,
STITCH :1186 and STITCH_PARTIAL :1187 (closed stitch), PREFILL_TOUCH :617,
PREFILL_STAGE / PREFILL_STAGE_GROUP_MB :1603-1608, GROUP_BYTES :1531;
``sync_from_environ()`` re-reads them (config.py:853).  FUSED_PREFILL
:1633 and ATTN_SUB_CHUNK :1562 for the fused prefill pass; PREFILL_AHEAD
:1583 for prefill-time prediction; FLOW / FLOW_WARMUP / FLOW_WARM_HIT
:1218-1237 and FLOW_MAX_CRIT :1253 for flow decode; PREDICT_DEPTH :747, PREDICT_SLACK :761 and
PREFETCH_DEPTH :722 for speculative prefetch (PREFETCH_DEPTH defaults to 0
here: the previous-token heuristic pays off with the reference's SSD queue,
not a PCIe copy engine); PREDICT and the governor knobs :735-741;
SLAB_VERIFY :1467 for the slot-safety ledger.  DECODE_MAX_TOKENS is the
reference's _DECODE_MAX_TOKENS (streaming.py:69): calls of more tokens take
the prefill residency policy.
"""

from __future__ import annotations

import os


def _env(name: str, default, cast):
    raw = os.environ.get("PAGED_MOE_" + name)
    if raw is None or raw == "":
        return default
    try:
        return cast(raw)
    except ValueError:
        return default


def _bool(v: str) -> bool:
    return v.strip().lower() not in ("0", "false", "off", "no")


SLAB_RESERVE_FRAC = 0.1   # slots held back from the resident budget
LFRU = True               # second-chance eviction for reused experts
LFRU_SCAN = 8             # entries scanned per eviction
STITCH = True             # pin every expert in a fixed slot when the slab holds them all
STITCH_PARTIAL = False    # closed stitch: one-pass decode over the live table, replayed on a miss
COPY_SPLIT_BYTES = 64 << 20  # H2D copy piece size (an expert of up to 64 MiB is one copy)
COPY_STREAMS = 2          # copy streams of the engine
DECODE_MAX_TOKENS = 20    # calls of more tokens are prefill (no touch, no eviction)
PREFILL_STAGE = True      # stage slots for prefill misses that find no free slot
PREFILL_STAGE_GROUP_MB = 384  # prefill fetch group size; the stage holds four groups
GROUP_BYTES = 1024 << 20  # ceiling on one prefill fetch group
FUSED_PREFILL = True      # long calls sub-chunk attention, run the MoE once
PREFILL_AHEAD = True      # a prefill layer starts the next layer's predicted reads
FLOW = False              # decode tokens with no host sync inside (residency once per token)
FLOW_WARMUP = 2           # tokens after a prefill that take the per-layer path first
FLOW_WARM_HIT = 0.9       # hit-rate EMA the per-layer path must reach before flow resumes
FLOW_MAX_CRIT = 5.0       # flow stops above this many missing routed experts per token (EMA)
PREDICT_DEPTH = 3         # route prediction: layers predicted ahead per stride
PREDICT_SLACK = 2         # extra experts per predicted layer beyond its top-k
PREFETCH_DEPTH = 0        # previous-token heuristic: next layers' last ids (0 = off)
PREDICT = "auto"          # route prediction: on, off, or auto (A/B governor decides)
PREDICT_WINDOW = 8        # governor: decode tokens per window
PREDICT_MIN_TOKENS = 96   # governor: tokens of evidence per state before deciding
PREDICT_MARGIN = 1.03     # governor: how much faster a state must measure
PREDICT_Z = 2.0           # governor: error bars the gap must also clear
PREDICT_MAX_PROBE = 6     # governor: inconclusive after this many times the evidence -> off
PREDICT_HOLD = 128        # governor: windows a decision is kept before re-probing
ATTN_SUB_CHUNK = 2048     # rows per attention sub-chunk, at most
ATTN_SCORE_MB = 1024      # fp32 score matrix (heads x rows x keys) of one sub-chunk, at most
SLAB_VERIFY = False       # replay copy/compute ordering per slot and flag races (debug)


def sync_from_environ() -> None:
    global SLAB_RESERVE_FRAC, LFRU, LFRU_SCAN, STITCH, STITCH_PARTIAL, COPY_SPLIT_BYTES
    global COPY_STREAMS
    global DECODE_MAX_TOKENS, PREFILL_STAGE, PREFILL_STAGE_GROUP_MB, GROUP_BYTES
    global FUSED_PREFILL, ATTN_SUB_CHUNK, ATTN_SCORE_MB, FLOW, FLOW_WARMUP, FLOW_WARM_HIT
    global PREFILL_AHEAD, FLOW_MAX_CRIT
    global PREDICT_DEPTH, PREDICT_SLACK, PREFETCH_DEPTH, PREDICT, PREDICT_WINDOW
    global PREDICT_MIN_TOKENS, PREDICT_MARGIN, PREDICT_Z, PREDICT_MAX_PROBE, PREDICT_HOLD
    global SLAB_VERIFY
    SLAB_RESERVE_FRAC = _env("SLAB_RESERVE_FRAC", 0.1, float)
    LFRU = _env("LFRU", True, _bool)
    LFRU_SCAN = _env("LFRU_SCAN", 8, int)
    STITCH = _env("STITCH", True, _bool)
    STITCH_PARTIAL = _env("STITCH_PARTIAL", False, _bool)
    COPY_SPLIT_BYTES = _env("COPY_SPLIT_KB", 65536, int) * 1024
    COPY_STREAMS = _env("COPY_STREAMS", 2, int)
    DECODE_MAX_TOKENS = _env("DECODE_MAX_TOKENS", 20, int)
    PREFILL_STAGE = _env("PREFILL_STAGE", True, _bool)
    PREFILL_STAGE_GROUP_MB = _env("PREFILL_STAGE_GROUP_MB", 384, int)
    GROUP_BYTES = _env("GROUP_MB", 1024, int) << 20
    FUSED_PREFILL = _env("FUSED_PREFILL", True, _bool)
    PREFILL_AHEAD = _env("PREFILL_AHEAD", True, _bool)
    ATTN_SUB_CHUNK = _env("ATTN_SUB_CHUNK", 2048, int)
    ATTN_SCORE_MB = _env("ATTN_SCORE_MB", 1024, int)
    FLOW = _env("FLOW", False, _bool)
    FLOW_WARMUP = _env("FLOW_WARMUP", 2, int)
    FLOW_WARM_HIT = _env("FLOW_WARM_HIT", 0.9, float)
    FLOW_MAX_CRIT = _env("FLOW_MAX_CRIT", 5.0, float)
    PREDICT_DEPTH = _env("PREDICT_DEPTH", 3, int)
    PREDICT_SLACK = _env("PREDICT_SLACK", 2, int)
    PREFETCH_DEPTH = _env("PREFETCH_DEPTH", 0, int)
    PREDICT = _env("PREDICT", "auto", str).strip().lower()
    PREDICT_WINDOW = _env("PREDICT_WINDOW", 8, int)
    PREDICT_MIN_TOKENS = _env("PREDICT_MIN_TOKENS", 96, int)
    PREDICT_MARGIN = _env("PREDICT_MARGIN", 1.03, float)
    PREDICT_Z = _env("PREDICT_Z", 2.0, float)
    PREDICT_MAX_PROBE = _env("PREDICT_MAX_PROBE", 6, int)
    PREDICT_HOLD = _env("PREDICT_HOLD", 128, int)
    SLAB_VERIFY = _env("SLAB_VERIFY", False, _bool)


sync_from_environ()
