"""torch-tensor wrappers over the libpmoe C ABI (one function per entry point).

Every function takes device tensors, checks dtype/shape/contiguity on the
host, and enqueues the HIP kernels on torch's current stream.  Packed
quantized words travel as ``torch.int32`` (same bits as the u32 of the
format); bf16 data as ``torch.bfloat16``.  There is no CPU path: without the
built library every call raises ``PmoeError``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import Geom, RouteCfg, check, lib

_WS: dict = {}
_MOE_WS: dict = {}
# Workspaces handed out before a larger call replaced them.  They are never
# freed: a HIP graph captured over an earlier call keeps their raw pointers,
# and a replay must not write into memory torch has given to another tensor.
_RETIRED: dict = {"dispatch": [], "MoE": []}
# Pinned host words the workspaces' error words are copied into at sync points.
_ERR_HOST: dict = {}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t, dtype, name, ndim=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a device tensor (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim} dims, got {tuple(t.shape)}")


def _grown(cache: dict, key, nbytes: int, device, what: str):
    """The cached buffer of at least nbytes, or a new one that replaces it
    (the old one is retired, not freed).  Growth is by at least 1.5x, so a
    sequence of larger calls retires only a few buffers.  Growing while the
    current stream is being captured into a graph raises: the capture would
    hold a pointer that a later, larger eager call cannot replace."""
    buf = cache.get(key)
    if buf is not None and buf.numel() >= nbytes:
        return buf, False
    if torch.cuda.is_current_stream_capturing():
        raise _lib.PmoeError(f"{what} workspace would grow to {nbytes} B during graph capture; "
                             "run the largest call once before capturing")
    size = max(int(nbytes), 256)
    if buf is not None:
        size = max(size, buf.numel() * 3 // 2)
        _RETIRED[what].append(buf)
    buf = torch.empty(size, dtype=torch.uint8, device=device)
    cache[key] = buf
    return buf, True


def workspace(nbytes: int, device) -> torch.Tensor:
    """A cached uint8 scratch tensor of at least nbytes on device."""
    return _grown(_WS, torch.device(device).index or 0, nbytes, device, "dispatch")[0]


# ---------------------------------------------------------------- routing

def router_logits(x: torch.Tensor, w: torch.Tensor, logit_bias=None) -> torch.Tensor:
    """fp32 logits [N, E] of x [N, D] bf16 against w [E, D] bf16."""
    _need(x, torch.bfloat16, "x", 2)
    _need(w, torch.bfloat16, "w", 2)
    n, d = x.shape
    e = w.shape[0]
    if w.shape[1] != d:
        raise ValueError("router weight hidden size mismatch")
    if logit_bias is not None:
        _need(logit_bias, torch.float32, "logit_bias", 1)
    out = torch.empty((n, e), dtype=torch.float32, device=x.device)
    check(lib().pmoe_router_logits(_ptr(x), _ptr(w), _ptr(logit_bias), n, d, e, _ptr(out),
                                   _stream()), "pmoe_router_logits")
    return out


def route_softmax_topk(logits: torch.Tensor, k: int, norm_topk_prob: bool = True):
    _need(logits, torch.float32, "logits", 2)
    n, e = logits.shape
    inds = torch.empty((n, k), dtype=torch.int32, device=logits.device)
    wts = torch.empty((n, k), dtype=torch.float32, device=logits.device)
    check(lib().pmoe_route_softmax_topk(_ptr(logits), n, e, k, int(bool(norm_topk_prob)),
                                        _ptr(inds), _ptr(wts), _stream()),
          "pmoe_route_softmax_topk")
    return inds, wts


def route_sigmoid_group_topk(logits, bias, n_group: int, topk_group: int, k: int,
                             norm_topk_prob: bool = True, routed_scale: float = 1.0):
    _need(logits, torch.float32, "logits", 2)
    _need(bias, torch.float32, "bias", 1)
    n, e = logits.shape
    inds = torch.empty((n, k), dtype=torch.int32, device=logits.device)
    wts = torch.empty((n, k), dtype=torch.float32, device=logits.device)
    check(lib().pmoe_route_sigmoid_group_topk(
        _ptr(logits), _ptr(bias), n, e, n_group, topk_group, k, int(bool(norm_topk_prob)),
        float(routed_scale), _ptr(inds), _ptr(wts), _stream()), "pmoe_route_sigmoid_group_topk")
    return inds, wts


# ---------------------------------------------------------------- dispatch

def dispatch(inds: torch.Tensor, n_experts: int) -> dict:
    """Stable grouping of the flat ids by expert (see pmoe_dispatch)."""
    _need(inds, torch.int32, "inds")
    rows = inds.numel()
    dev = inds.device
    out = {
        "order": torch.empty(rows, dtype=torch.int32, device=dev),
        "counts": torch.empty(n_experts, dtype=torch.int32, device=dev),
        "offsets": torch.empty(n_experts + 1, dtype=torch.int32, device=dev),
        "inv": torch.empty(rows, dtype=torch.int32, device=dev),
        "active": torch.empty(n_experts, dtype=torch.int32, device=dev),
        "n_active": torch.empty(1, dtype=torch.int32, device=dev),
    }
    wsb = lib().pmoe_dispatch_workspace(rows, n_experts)
    ws = workspace(wsb, dev)
    check(lib().pmoe_dispatch(_ptr(inds), rows, n_experts, _ptr(out["order"]),
                              _ptr(out["counts"]), _ptr(out["offsets"]), _ptr(out["inv"]),
                              _ptr(out["active"]), _ptr(out["n_active"]), _ptr(ws), ws.numel(),
                              _stream()), "pmoe_dispatch")
    return out


# ---------------------------------------------------------------- format

def quantize(w: torch.Tensor, bits: int, group: int = 64, out=None):
    """fp32 [R, C] -> (q int32 [R, C*bits/32], scales bf16, biases bf16).
    ``out`` = (q, s, b) contiguous tensors to write into (e.g. slab views)."""
    _need(w, torch.float32, "w", 2)
    r, c = w.shape
    if c % group or (c * bits) % 32:
        raise ValueError("columns must be a multiple of the group size")
    if out is None:
        q = torch.empty((r, c * bits // 32), dtype=torch.int32, device=w.device)
        s = torch.empty((r, c // group), dtype=torch.bfloat16, device=w.device)
        b = torch.empty((r, c // group), dtype=torch.bfloat16, device=w.device)
    else:
        q, s, b = out
        for t, dt, shape, name in ((q, torch.int32, (r, c * bits // 32), "q"),
                                   (s, torch.bfloat16, (r, c // group), "scales"),
                                   (b, torch.bfloat16, (r, c // group), "biases")):
            _need(t, dt, name)
            if tuple(t.shape) != shape:
                raise ValueError(f"{name}: expected {shape}, got {tuple(t.shape)}")
    check(lib().pmoe_quantize(_ptr(w), r, c, bits, group, _ptr(q), _ptr(s), _ptr(b), _stream()),
          "pmoe_quantize")
    return q, s, b


def dequant(q, scales, biases, bits: int, group: int = 64) -> torch.Tensor:
    _need(q, torch.int32, "q", 2)
    _need(scales, torch.bfloat16, "scales", 2)
    _need(biases, torch.bfloat16, "biases", 2)
    r = q.shape[0]
    c = q.shape[1] * 32 // bits
    out = torch.empty((r, c), dtype=torch.bfloat16, device=q.device)
    check(lib().pmoe_dequant(_ptr(q), _ptr(scales), _ptr(biases), r, c, bits, group, _ptr(out),
                             _stream()), "pmoe_dequant")
    return out


# ---------------------------------------------------------------- experts

def moe_workspace(g: Geom, n: int, k: int, shared: int, n_experts: int, device,
                  fresh: bool = False) -> torch.Tensor:
    """Workspace of the expert entry points (pmoe_moe_workspace bytes).  Its
    synchronisation header is zeroed on allocation (pmoe_moe_workspace_init);
    the cached buffer is separate from the dispatch scratch so nothing else
    ever writes the header.  fresh=True returns a new, private buffer."""
    nb = max(int(lib().pmoe_moe_workspace(ctypes.byref(g), n, k, shared, n_experts)), 256)
    if fresh:
        buf = torch.empty(nb, dtype=torch.uint8, device=device)
        check(lib().pmoe_moe_workspace_init(_ptr(buf), buf.numel(), _stream()),
              "pmoe_moe_workspace_init")
        return buf
    buf, new = _grown(_MOE_WS, torch.device(device).index or 0, nb, device, "MoE")
    if new:
        check(lib().pmoe_moe_workspace_init(_ptr(buf), buf.numel(), _stream()),
              "pmoe_moe_workspace_init")
    return buf


def _live_moe_workspaces():
    return list(_MOE_WS.values()) + _RETIRED["MoE"]


def note_workspace_errors() -> None:
    """Enqueue, on the current stream, copies of every cached MoE
    workspace's error word into pinned host memory (no wait).  A caller that
    synchronises the stream next reads them with ``raise_workspace_errors``."""
    for ws in _live_moe_workspaces():
        host = _ERR_HOST.get(ws.data_ptr())
        if host is None:
            host = _ERR_HOST[ws.data_ptr()] = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        check(lib().pmoe_moe_workspace_error_async(_ptr(ws), _ptr(host), _stream()),
              "pmoe_moe_workspace_error_async")


def raise_workspace_errors() -> None:
    """After a stream sync that followed ``note_workspace_errors``: raise
    PmoeError if a grid barrier of the one-launch decode timed out (those
    layer outputs are NaN).  The failed workspace is re-initialised first,
    so the next call runs normally."""
    words = {ws.data_ptr(): int(_ERR_HOST.get(ws.data_ptr(),
                                              torch.zeros(1, dtype=torch.int32))[0])
             for ws in _live_moe_workspaces()}
    bad = [ws for ws in _live_moe_workspaces() if words[ws.data_ptr()] != 0]
    if not bad:
        return
    err = 0
    for ws in bad:
        err |= words[ws.data_ptr()]
        _ERR_HOST[ws.data_ptr()].zero_()
        check(lib().pmoe_moe_workspace_init(_ptr(ws), ws.numel(), _stream()),
              "pmoe_moe_workspace_init")
    what = []
    if err & 1:
        what.append("a barrier wait timed out (a block was not resident in time)")
    if err & 2:
        what.append("the blocks of one group of the expert-per-XCD launch ran on "
                    "different XCDs")
    raise _lib.PmoeError("one-launch decode: " + "; ".join(what or [f"error word {err:#x}"])
                         + "; the affected layer outputs are NaN")


def check_workspace_errors() -> None:
    """Synchronising form of note + raise, for sync points of their own
    (get_stats)."""
    note_workspace_errors()
    torch.cuda.current_stream().synchronize()
    raise_workspace_errors()


def set_split_probe(on: bool) -> None:
    """Debug: make the expert-per-XCD decode's group 0 look split across two
    XCDs (pmoe_set_split_probe), so its placement check fires."""
    check(lib().pmoe_set_split_probe(int(bool(on))), "pmoe_set_split_probe")


def set_barrier_spin(ticks: int) -> None:
    """Debug: grid-barrier poll limit of later one-launch decode calls in
    100 MHz ticks (0 = the default 0.5 s); see pmoe_set_barrier_spin."""
    check(lib().pmoe_set_barrier_spin(int(ticks)), "pmoe_set_barrier_spin")


def workspace_error(ws: torch.Tensor) -> int:
    """The sticky error word of a MoE workspace header (synchronises)."""
    err = ctypes.c_uint32()
    check(lib().pmoe_moe_workspace_status(_ptr(ws), ctypes.byref(err), _stream()),
          "pmoe_moe_workspace_status")
    return int(err.value)


def _table_ptr(table):
    if isinstance(table, torch.Tensor):
        _need(table, torch.int32, "table", 1)
        return _ptr(table)
    return ctypes.c_void_p(int(table))


def switch_glu(g: Geom, slab: torch.Tensor, table, n_experts: int, x: torch.Tensor,
               inds: torch.Tensor) -> torch.Tensor:
    """y [N, K, D] bf16: row (n, k) through the expert in slot table[inds[n, k]]."""
    _need(x, torch.bfloat16, "x", 2)
    _need(inds, torch.int32, "inds", 2)
    n, k = inds.shape
    if x.shape != (n, g.hidden):
        raise ValueError(f"x must be [{n}, {g.hidden}], got {tuple(x.shape)}")
    y = torch.empty((n, k, g.hidden), dtype=torch.bfloat16, device=x.device)
    ws = moe_workspace(g, n, k, 0, n_experts, x.device)
    check(lib().pmoe_switch_glu(ctypes.byref(g), _ptr(slab), _table_ptr(table), n_experts,
                                _ptr(x), _ptr(inds), n, k, _ptr(y), _ptr(ws), ws.numel(),
                                _stream()), "pmoe_switch_glu")
    return y


def count_missing(table, ids: torch.Tensor, n_experts: int, counter: torch.Tensor) -> None:
    """counter (device int32 [1]) += routed ids of ``ids`` that ``table``
    (device int32 [E], a tensor or a device address) maps to no slot."""
    _need(ids, torch.int32, "ids")
    _need(counter, torch.int32, "counter", 1)
    check(lib().pmoe_count_missing(_table_ptr(table), _ptr(ids), ids.numel(), n_experts,
                                   _ptr(counter), _stream()), "pmoe_count_missing")


def moe_experts(g: Geom, slab, table, n_experts: int, x, inds, weights, shared_slot: int = -1,
                shared_gate=None) -> torch.Tensor:
    """out [N, D] bf16 = sum_k w[n,k] FFN_{inds[n,k]}(x[n]) (+ shared)."""
    _need(x, torch.bfloat16, "x", 2)
    _need(inds, torch.int32, "inds", 2)
    _need(weights, torch.float32, "weights", 2)
    n, k = inds.shape
    out = torch.empty((n, g.hidden), dtype=torch.bfloat16, device=x.device)
    ws = moe_workspace(g, n, k, int(shared_slot >= 0), n_experts, x.device)
    check(lib().pmoe_moe_experts(ctypes.byref(g), _ptr(slab), _table_ptr(table), n_experts,
                                 _ptr(x), _ptr(inds), _ptr(weights), n, k, int(shared_slot),
                                 _ptr(shared_gate), _ptr(out), _ptr(ws), ws.numel(), _stream()),
          "pmoe_moe_experts")
    return out


def combine(y: torch.Tensor, weights: torch.Tensor, shared_y=None, shared_logit=None):
    """out [N, D] bf16 = sum_k weights[n,k] y[n,k] (+ s * shared_y[n]) with
    fp32 accumulation in k order; s = 1 or sigmoid(shared_logit[n])."""
    _need(y, torch.bfloat16, "y", 3)
    _need(weights, torch.float32, "weights", 2)
    n, k, d = y.shape
    if tuple(weights.shape) != (n, k):
        raise ValueError(f"weights must be [{n}, {k}], got {tuple(weights.shape)}")
    if shared_y is not None:
        _need(shared_y, torch.bfloat16, "shared_y", 2)
        if tuple(shared_y.shape) != (n, d):
            raise ValueError("shared_y must be [N, D]")
    if shared_logit is not None:
        _need(shared_logit, torch.float32, "shared_logit")
        if shared_logit.numel() != n:
            raise ValueError("shared_logit must hold N values")
    out = torch.empty((n, d), dtype=torch.bfloat16, device=y.device)
    check(lib().pmoe_combine(_ptr(y), _ptr(weights), n, k, d, _ptr(shared_y), _ptr(shared_logit),
                             _ptr(out), _stream()), "pmoe_combine")
    return out


def route_cfg(scoring: str, n_experts: int, top_k: int, norm_topk_prob: bool = True,
              n_group: int = 1, topk_group: int = 1, routed_scale: float = 1.0) -> RouteCfg:
    rc = RouteCfg()
    rc.scoring = _lib.SCORE_SOFTMAX if scoring == "softmax" else _lib.SCORE_SIGMOID
    rc.n_experts = n_experts
    rc.top_k = top_k
    rc.norm_topk_prob = int(bool(norm_topk_prob))
    rc.n_group = n_group
    rc.topk_group = topk_group
    rc.routed_scale = float(routed_scale)
    return rc


def moe_block(g: Geom, rc: RouteCfg, slab, table, gate_w, x, score_bias=None, logit_bias=None,
              shared_slot: int = -1, shared_gate=None, out=None, inds=None, weights=None,
              ws=None):
    """Route -> dispatch -> experts -> combine in one call.  Returns
    (out [N, D] bf16, inds [N, K] int32, weights [N, K] fp32)."""
    _need(x, torch.bfloat16, "x", 2)
    _need(gate_w, torch.bfloat16, "gate_w", 2)
    n = x.shape[0]
    k = rc.top_k
    dev = x.device
    if out is None:
        out = torch.empty((n, g.hidden), dtype=torch.bfloat16, device=dev)
    if inds is None:
        inds = torch.empty((n, k), dtype=torch.int32, device=dev)
    if weights is None:
        weights = torch.empty((n, k), dtype=torch.float32, device=dev)
    if ws is None:
        ws = moe_workspace(g, n, k, int(shared_slot >= 0), rc.n_experts, dev)
    check(lib().pmoe_moe_block(ctypes.byref(g), ctypes.byref(rc), _ptr(slab), _table_ptr(table),
                               _ptr(gate_w), _ptr(score_bias), _ptr(logit_bias), _ptr(x), n,
                               int(shared_slot), _ptr(shared_gate), _ptr(out), _ptr(inds),
                               _ptr(weights), _ptr(ws), ws.numel(), _stream()), "pmoe_moe_block")
    return out, inds, weights
