"""The MoE seam and the blocks around it (torch modules over libpmoe).

Mirrors the reference's drop-in surface (streaming.py):
  * ``StreamedSwitchGLU.__call__(x, indices) -> [..., K, D]`` -- per-slot,
    uncombined expert outputs in ``indices`` order, the contract of mlx-lm's
    ``SwitchGLU`` that the reference replaces (streaming.py:946-1401);
  * ``patch_model(model, cache)`` swaps every resident ``QuantizedSwitchGLU``
    for a ``StreamedSwitchGLU`` backed by the expert cache
    (streaming.py:2575-2688); ``find_switch_glus`` (:2512-2526);
  * the MoE blocks that call it: softmax top-k (Qwen3-MoE / Qwen3-Next, with an
    optional gated shared expert) and sigmoid grouped top-k (DeepSeek-V3 /
    Kimi-K2, with a shared expert) -- router, top-k, experts and the fixed-order
    combine run as HIP kernels (pmoe_moe_block).
All compute is on the GPU; there is no CPU path.
"""

from __future__ import annotations

import torch
from torch import nn

from . import config
from . import kernels as K
from ._lib import geom as make_geom
from .cache import ExpertCache
from .ring import PrefetchRing
from .slab import SlabStore

PROJS = ("gate_proj", "up_proj", "down_proj")


class QuantizedSwitchGLU(nn.Module):
    """Resident stacked experts: E affine-quantized SwiGLU experts (plus an
    optional shared expert in slot E) in one slab, expert e in slot e.  The
    resident counterpart of mlx-lm's SwitchGLU over QuantizedSwitchLinear."""

    def __init__(self, hidden: int, inter: int, n_experts: int, bits: int = 4, group: int = 64,
                 n_shared: int = 0, device="cuda"):
        super().__init__()
        self.geom = make_geom(hidden, inter, bits, group)
        self.hidden, self.inter, self.bits = hidden, inter, bits
        self.n_experts = n_experts
        self.n_shared = n_shared
        self.slab = SlabStore(self.geom, n_experts + n_shared, device)
        self.register_buffer("table", torch.arange(n_experts, dtype=torch.int32, device=device),
                             persistent=False)

    @property
    def shared_slot(self) -> int:
        return self.n_experts if self.n_shared else -1

    def quantize_expert(self, e: int, gate_w, up_w, down_w) -> None:
        """Quantize fp32 weights gate/up [I, D], down [D, I] into expert e's
        slot (e == n_experts: the shared expert)."""
        for proj, w in zip(PROJS, (gate_w, up_w, down_w)):
            self.slab.quantize_into(e, proj, w.float().contiguous())

    def load_expert(self, e: int, comps: dict) -> None:
        """Copy already quantized components (name -> tensor/array) into slot e."""
        self.slab.write_expert(e, comps)

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        lead = indices.shape
        x2 = x.reshape(-1, self.hidden).to(torch.bfloat16).contiguous()
        ind2 = indices.reshape(-1, lead[-1]).to(torch.int32).contiguous()
        y = K.switch_glu(self.geom, self.slab.buf, self.table, self.n_experts, x2, ind2)
        return y.reshape(*lead, self.hidden)


class StreamedSwitchGLU(nn.Module):
    """The seam: same call contract as QuantizedSwitchGLU, experts paged
    into the cache's slab on demand.

    With every expert stitched into a fixed slot the call never leaves the
    GPU.  Otherwise the routed ids reach the host (the one sync per layer the
    reference also pays, streaming.py:1103-1129), the cache copies the misses
    from the pinned host store and publishes the expert->slot table, and the
    expert kernels read the slab through that table.

    Calls of at most ``config.DECODE_MAX_TOKENS`` tokens use the decode
    residency policy (hits move to MRU, misses may evict).  Longer calls are
    prefill (streaming.py:1313+, cache.py:2535-2578): fetch groups that never
    evict and leave the decode hot set's recency alone, each group's copies
    issued while the previous group computes."""

    def __init__(self, layer_key, original: QuantizedSwitchGLU | None, cache: ExpertCache,
                 ring=None, predictor=None):
        super().__init__()
        self.layer_key = layer_key
        self.cache = cache
        self.ring = ring
        self.ring_index = -1
        self.pred = predictor
        g = cache.geom
        self.hidden, self.inter, self.bits = g.hidden, g.inter, g.bits
        self.n_experts = cache.n_experts
        self.last_ids: list[int] = []
        # prefill fetch groups of the last call: the first group's ids, then
        # ("open" | "after_done", ids) for each later group -- requested while
        # the previous group still held its slots, or after it gave them back
        self.last_groups: list = []

    @property
    def geom(self):
        return self.cache.geom

    def routed_ids(self, indices: torch.Tensor) -> list:
        """The layer's distinct routed ids, ascending (one host sync).  The
        sync also carries the MoE workspaces' error words: a timed-out grid
        barrier of an earlier one-launch decode raises here."""
        K.note_workspace_errors()
        ids = [e for e in torch.unique(indices.reshape(-1)).tolist() if 0 <= e < self.n_experts]
        K.raise_workspace_errors()
        if self.ring is not None:
            self.ring.collect_predictions()   # they rode this sync
        return ids

    def plan_groups(self, indices: torch.Tensor) -> list:
        """Decode-policy fetch groups: the distinct routed ids split into
        groups that each fit the slab's routed slots, already resident ids
        first so they are not evicted by their own layer.  One group is the
        normal case; several happen only when a decode call routes to more
        experts than the slab holds."""
        ids = self.routed_ids(indices)
        cap = self.cache.routed_slots
        if len(ids) <= cap:
            return [ids]
        table = self.cache.host_table(self.layer_key)
        ordered = [e for e in ids if table[e] >= 0] + [e for e in ids if table[e] < 0]
        return [sorted(ordered[i:i + cap]) for i in range(0, len(ordered), cap)]

    def passes(self, indices: torch.Tensor, x2: torch.Tensor | None = None):
        """Make the routed experts resident, one fetch group at a time.
        Yields (member ids, or None when this pass covers every routed id;
        device table pointer); the caller enqueues the pass's compute before
        resuming the generator, and must run it to the end.  ``x2`` (the
        call's rows) feeds prefill-time prediction of the next layer."""
        c, lk = self.cache, self.layer_key
        if c.stitched:
            yield None, c.table_ptr(lk)
            return
        n_tokens = indices.reshape(-1, indices.shape[-1]).shape[0]
        if n_tokens <= config.DECODE_MAX_TOKENS:
            yield from self._decode_passes(self.plan_groups(indices))
        else:
            if self.ring is not None:
                self.ring.predict_prefill(self.ring_index, x2)
            yield from self._prefill_passes(self.routed_ids(indices))
            if self.ring is not None:
                self.ring.settle_prefill_ahead(self.ring_index)

    def _decode_passes(self, groups):
        c, lk = self.cache, self.layer_key
        if self.ring is not None:
            self.ring.note_demand(self.ring_index, [e for grp in groups for e in grp])
        for grp in groups:
            c.fetch(lk, grp)
            c.spec_fence()        # guesses issued after this compute may run under it
            yield (None if len(groups) == 1 else grp), c.table_ptr(lk)
        c.group_passes += len(groups) - 1
        self.last_ids = [e for grp in groups for e in grp]

    def _prefill_passes(self, ids):
        """Prefill fetch groups: resident ids (hits) ride with the first
        group; the misses are cut into groups no larger than the stage's
        group size and the free + stage slots left.  Group i+1's policy step
        and copies are issued right after group i's compute is enqueued, so
        they run under it; its copies wait only for the compute before
        group i (the slots group i holds are not handed out until then)."""
        c, lk = self.cache, self.layer_key
        table = c.host_table(lk)
        hits = [e for e in ids if table[e] >= 0]
        pending = [e for e in ids if table[e] < 0]
        per = int(c.geom.expert_bytes)
        group_max = max(1, min(config.GROUP_BYTES,
                               max(config.PREFILL_STAGE_GROUP_MB << 20, 8 * per)) // per)

        def take():
            free, stage, _ = c.capacity()
            n = min(group_max, free + stage, len(pending))
            grp = pending[:n]
            del pending[:n]
            return grp

        c.fence()
        first = hits + take()
        if pending and len(first) == len(hits):
            # no free or stage slot at all: the decode policy (which evicts)
            # for every miss
            yield from self._decode_passes([hits] + self._cut(pending) if hits else
                                           self._cut(pending))
            return
        cur = c.fetch_prefill(lk, first)
        self.last_groups = [cur.ids]
        single = not pending
        if single and self.ring is not None:
            self.ring.issue_prefill_ahead(self.ring_index)   # every read of this layer is queued
        n_pass = 0
        while cur is not None:
            c.publish_group(cur)
            c.join()
            c.fence()
            yield (None if single else cur.ids), c.table_ptr(lk)
            n_pass += 1
            nxt = None
            if pending:
                grp = take()
                if not grp:
                    # the current group holds every slot left: it goes back
                    # first, and the next copies wait for its compute
                    c.prefill_done(cur)
                    cur = None
                    c.fence()
                    grp = take()
                if grp:
                    nxt = c.fetch_prefill(lk, grp)
                    self.last_groups.append(("after_done" if cur is None else "open", nxt.ids))
                    if not pending and self.ring is not None:
                        self.ring.issue_prefill_ahead(self.ring_index)
            if cur is not None:
                c.prefill_done(cur)
            cur = nxt
        c.sync_table(lk)
        c.group_passes += n_pass - 1
        self.last_ids = list(ids)

    def _cut(self, ids):
        cap = self.cache.routed_slots
        return [ids[i:i + cap] for i in range(0, len(ids), cap)]

    def run_passes(self, ind2: torch.Tensor, compute, x2: torch.Tensor | None = None) -> torch.Tensor:
        """Per-slot outputs [N, K, D] over every pass of ``passes``:
        ``compute(ids, table)`` runs one pass.  A pass over a subset of the
        routed ids sees the others dropped to -1 (zero rows), and its rows are
        merged by selection, so every row is bit-identical to a single pass
        over a slab that holds every routed expert."""
        y = None
        for member, table in self.passes(ind2, x2):
            if member is None:
                y = compute(ind2, table)
                self.cache.note_compute(self.layer_key)
                continue
            keep = torch.isin(ind2, torch.tensor(member, dtype=torch.int32, device=ind2.device))
            y_g = compute(torch.where(keep, ind2, torch.full_like(ind2, -1)), table)
            self.cache.note_compute(self.layer_key)
            y = y_g if y is None else torch.where(keep[..., None], y_g, y)
        return y

    def graph_mode(self, n_tokens: int):
        """Enter this layer's call on the ring: "flow" (a flow token),
        "closed" (a closed-stitch attempt) or None (the per-layer path)."""
        if self.ring is None:
            return None
        return self.ring.layer_call(self.ring_index, n_tokens)

    def call(self, x2: torch.Tensor, ind2: torch.Tensor, compute) -> torch.Tensor:
        """One seam call over flat rows x2 [N, D] and routing ind2 [N, K]:
        a flow token or a closed-stitch attempt computes once against the
        device table published at the token's start (no host round trip;
        non-resident experts give zero rows -- a closed attempt also counts
        them on the device); otherwise every fetch pass of ``run_passes``,
        then speculation for the layers ahead.  ``compute(ids, table)``
        enqueues the expert kernels of one pass."""
        c = self.cache
        mode = None if c.stitched else self.graph_mode(ind2.shape[0])
        if mode is not None:
            table = c.table_ptr(self.layer_key)
            y = compute(ind2, table)
            c.note_compute(self.layer_key)
            if mode == "flow":
                self.ring.note(self.ring_index, ind2)
            else:
                self.ring.count_missing(table, ind2)
            return y
        y = self.run_passes(ind2, compute, x2)
        if self.ring is not None and ind2.shape[0] <= config.DECODE_MAX_TOKENS:
            self.ring.speculate(self.ring_index, x2)
        return y

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        lead = indices.shape
        x2 = x.reshape(-1, self.hidden).to(torch.bfloat16).contiguous()
        ind2 = indices.reshape(-1, lead[-1]).to(torch.int32).contiguous()
        c = self.cache
        y = self.call(x2, ind2, lambda ids, table: K.switch_glu(
            c.geom, c.slab.buf, table, self.n_experts, x2, ids))
        return y.reshape(*lead, self.hidden)


def _experts_of(switch_mlp):
    """(geom, slab tensor, table, n_experts, shared slot) of a resident or
    streamed switch."""
    if isinstance(switch_mlp, StreamedSwitchGLU):
        c = switch_mlp.cache
        return c.geom, c.slab.buf, None, c.n_experts, c.shared_slot(switch_mlp.layer_key)
    return (switch_mlp.geom, switch_mlp.slab.buf, switch_mlp.table, switch_mlp.n_experts,
            switch_mlp.shared_slot)


class _MoEBlock(nn.Module):
    scoring = "softmax"

    def _route_cfg(self):
        raise NotImplementedError

    def _score_bias(self):
        return None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
        g, slab, table, n_exp, shared_slot = _experts_of(self.switch_mlp)
        if not self.use_shared:
            shared_slot = -1
        rc = self._route_cfg()
        sg = self.shared_expert_gate if self.use_shared else None
        sm = self.switch_mlp
        mode = (sm.graph_mode(x2.shape[0])
                if isinstance(sm, StreamedSwitchGLU) and not sm.cache.stitched else None)
        if mode is not None:
            # flow token or closed-stitch attempt: the whole block on the GPU
            # against the device table published at the token's start
            # (streaming.py:675-724, :905-935)
            tab = sm.cache.table_ptr(sm.layer_key)
            out, inds, w = K.moe_block(g, rc, slab, tab, self.gate_weight, x2,
                                       score_bias=self._score_bias(), logit_bias=self.logit_bias,
                                       shared_slot=shared_slot, shared_gate=sg)
            sm.cache.note_compute(sm.layer_key)
            if mode == "flow":
                sm.ring.note(sm.ring_index, inds)
            else:
                sm.ring.count_missing(tab, inds)
            self.last_routing = (inds, w)
            return out.reshape(shape)
        if isinstance(sm, StreamedSwitchGLU) and not sm.cache.stitched:
            # route, then make the routed experts resident, then compute
            logits = K.router_logits(x2, self.gate_weight, self.logit_bias)
            if self.scoring == "softmax":
                inds, w = K.route_softmax_topk(logits, self.top_k, self.norm_topk_prob)
            else:
                inds, w = K.route_sigmoid_group_topk(logits, self._score_bias(), self.n_group,
                                                     self.topk_group, self.top_k,
                                                     self.norm_topk_prob, self.routed_scale)
            out = None
            y = None
            decode = x2.shape[0] <= config.DECODE_MAX_TOKENS
            for member, tab in sm.passes(inds, x2):
                if member is None and decode:
                    # every routed expert is resident: the one-launch block
                    # (it routes again, to the same bits), the same arithmetic
                    # as a flow token or a closed-stitch attempt
                    out = K.moe_block(g, rc, slab, tab, self.gate_weight, x2,
                                      score_bias=self._score_bias(), logit_bias=self.logit_bias,
                                      shared_slot=shared_slot, shared_gate=sg)[0]
                    sm.cache.note_compute(sm.layer_key)
                    continue
                if member is None:
                    out = K.moe_experts(g, slab, tab, n_exp, x2, inds, w, shared_slot, sg)
                    sm.cache.note_compute(sm.layer_key)
                    continue
                keep = torch.isin(inds, torch.tensor(member, dtype=torch.int32, device=x2.device))
                y_g = K.switch_glu(g, slab, tab, n_exp, x2,
                                   torch.where(keep, inds, torch.full_like(inds, -1)))
                sm.cache.note_compute(sm.layer_key)
                y = y_g if y is None else torch.where(keep[..., None], y_g, y)
            if out is None:
                shared_y = shared_logit = None
                if shared_slot >= 0:
                    one = torch.full((1,), shared_slot, dtype=torch.int32, device=x2.device)
                    zero = torch.zeros((x2.shape[0], 1), dtype=torch.int32, device=x2.device)
                    shared_y = K.switch_glu(g, slab, one, 1, x2, zero).reshape(x2.shape)
                    if sg is not None:
                        shared_logit = K.router_logits(x2, sg.reshape(1, -1)).reshape(-1)
                out = K.combine(y, w, shared_y, shared_logit)
            if sm.ring is not None and x2.shape[0] <= config.DECODE_MAX_TOKENS:
                sm.ring.speculate(sm.ring_index, x2)
            self.last_routing = (inds, w)
            return out.reshape(shape)
        if table is None:
            table = sm.cache.table_ptr(sm.layer_key)
        out, inds, w = K.moe_block(g, rc, slab, table, self.gate_weight, x2,
                                   score_bias=self._score_bias(), logit_bias=self.logit_bias,
                                   shared_slot=shared_slot, shared_gate=sg)
        self.last_routing = (inds, w)
        return out.reshape(shape)


def _predict_ids_softmax(blk, x, slack):
    logits = K.router_logits(x, blk.gate_weight, blk.logit_bias)
    m = min(blk.top_k + max(0, slack), 16, blk.gate_weight.shape[0])
    return K.route_softmax_topk(logits, m, False)[0]


class SoftmaxMoEBlock(_MoEBlock):
    """Qwen3-MoE / Qwen3-Next sparse MoE block: softmax router, top-k,
    optional renormalisation, optional shared expert scaled by
    sigmoid(x . shared_expert_gate).  ``logit_bias`` ([E] fp32) is an additive
    router-logit skew used by the uneven-load synthetic workloads."""

    scoring = "softmax"

    def __init__(self, gate_weight: torch.Tensor, switch_mlp, top_k: int,
                 norm_topk_prob: bool = True, shared_expert_gate: torch.Tensor | None = None,
                 use_shared: bool | None = None, logit_bias: torch.Tensor | None = None):
        super().__init__()
        self.gate_weight = gate_weight.to(torch.bfloat16).contiguous()
        self.switch_mlp = switch_mlp
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.shared_expert_gate = (None if shared_expert_gate is None
                                   else shared_expert_gate.to(torch.bfloat16).contiguous())
        has_shared = _experts_of(switch_mlp)[4] >= 0
        self.use_shared = has_shared if use_shared is None else use_shared
        self.logit_bias = logit_bias

    def _route_cfg(self):
        return K.route_cfg("softmax", self.gate_weight.shape[0], self.top_k, self.norm_topk_prob)

    def predict_ids(self, x, slack: int = 0):
        """This block's router on another layer's hidden state: top-(k +
        slack) ids (softmax is monotonic, so the top of the logits), device
        int32 [N, k + slack]; route prediction (streaming.py:2069-2110)."""
        return _predict_ids_softmax(self, x, slack)


class SigmoidGroupMoEBlock(_MoEBlock):
    """DeepSeek-V3 / Kimi-K2 MoE block: sigmoid scores plus
    e_score_correction_bias, grouped top-k, routed scaling, and an always-on
    shared expert (out = routed mixture + shared(x))."""

    scoring = "sigmoid"

    def __init__(self, gate_weight: torch.Tensor, e_score_correction_bias: torch.Tensor, switch_mlp,
                 top_k: int, n_group: int, topk_group: int, routed_scaling_factor: float,
                 norm_topk_prob: bool = True, use_shared: bool | None = None):
        super().__init__()
        self.gate_weight = gate_weight.to(torch.bfloat16).contiguous()
        self.e_score_correction_bias = e_score_correction_bias.float().contiguous()
        self.switch_mlp = switch_mlp
        self.top_k = top_k
        self.n_group = n_group
        self.topk_group = topk_group
        self.routed_scale = routed_scaling_factor
        self.norm_topk_prob = norm_topk_prob
        self.shared_expert_gate = None
        has_shared = _experts_of(switch_mlp)[4] >= 0
        self.use_shared = has_shared if use_shared is None else use_shared
        self.logit_bias = None

    def _score_bias(self):
        return self.e_score_correction_bias

    def _route_cfg(self):
        return K.route_cfg("sigmoid", self.gate_weight.shape[0], self.top_k, self.norm_topk_prob,
                           self.n_group, self.topk_group, self.routed_scale)

    def predict_ids(self, x, slack: int = 0):
        """Route prediction with this block's grouped top-k (the router
        returns the selected ids, streaming.py:2046-2068); slack widens the
        final top-k within the kept groups."""
        logits = K.router_logits(x, self.gate_weight, self.logit_bias)
        e = self.gate_weight.shape[0]
        m = min(self.top_k + max(0, slack), 16, (e // self.n_group) * self.topk_group)
        return K.route_sigmoid_group_topk(logits, self.e_score_correction_bias, self.n_group,
                                          self.topk_group, m, True, 1.0)[0]


# ---------------------------------------------------------------- model surgery

def _layer_order(path: str) -> tuple:
    """Sort key of a module path: its integer components in order
    ("model.layers.12.mlp.switch_mlp" -> (12,)), so layers sort numerically
    and paths without an index come first."""
    return tuple(int(p) for p in path.split(".") if p.isdecimal())


def find_switch_glus(model: nn.Module):
    """[(path, module)] of every QuantizedSwitchGLU in ``model``, in layer
    order (replaces streaming.py:2512-2526)."""
    found = [(p, m) for p, m in model.named_modules() if isinstance(m, QuantizedSwitchGLU)]
    return sorted(found, key=lambda pm: _layer_order(pm[0]))


def _swap_module(model: nn.Module, path: str, new: nn.Module) -> None:
    """Put ``new`` where ``path`` names a submodule.  nn.Module registers a
    child under its attribute name and nn.ModuleList under the decimal index
    string, so one setattr on the parent covers both."""
    parent_path, _, name = path.rpartition(".")
    parent = model.get_submodule(parent_path) if parent_path else model
    setattr(parent, name, new)


def build_cache_for(model: nn.Module, slots: int, model_path=None, **kw) -> ExpertCache:
    """An ExpertCache (with a pinned host store holding every expert of every
    QuantizedSwitchGLU of ``model``) for patch_model.  With ``model_path``
    the store is read from that quantized safetensors checkpoint (its MoE
    layers in layer order, one per module; checkpoint.py) instead of from the
    modules' own slabs -- the reference pages experts from the checkpoint
    files (safetensors_index.py)."""
    from .cache import HostExpertStore

    glus = find_switch_glus(model)
    if not glus:
        raise ValueError("no QuantizedSwitchGLU modules found")
    first = glus[0][1]
    n_shared = first.n_shared
    g = first.geom
    for _, m in glus:
        if (m.hidden, m.inter, m.bits, m.n_experts, m.n_shared) != (
                first.hidden, first.inter, first.bits, first.n_experts, n_shared):
            raise ValueError("all MoE layers must share one expert shape")
    if model_path is not None:
        store = HostExpertStore.from_checkpoint(model_path)
        sg = store.geom
        if (store.n_layers, store.n_experts, sg.hidden, sg.inter, sg.bits) != (
                len(glus), first.n_experts, first.hidden, first.inter, first.bits):
            store.close()
            raise ValueError(f"{model_path}: {store.n_layers} MoE layers of {store.n_experts} "
                             f"experts ({sg.hidden}/{sg.inter}/{sg.bits}-bit) do not match the "
                             f"model's {len(glus)} layers of {first.n_experts} "
                             f"({first.hidden}/{first.inter}/{first.bits}-bit)")
    else:
        store = HostExpertStore(g, len(glus), first.n_experts)
        for li, (_, m) in enumerate(glus):
            for e in range(m.n_experts):
                store.write_from_slot(li, e, m.slab, e)
    cache = ExpertCache(g, slots, [p for p, _ in glus], first.n_experts, host_store=store,
                        n_shared=n_shared, **kw)
    for li, (p, m) in enumerate(glus):
        if n_shared:
            cache.slab.slot_bytes(cache.shared_slot(p)).copy_(m.slab.slot_bytes(m.n_experts))
    return cache


def patch_model(model: nn.Module, cache: ExpertCache, tensor_index=None, prefetch_depth: int = 0,
                predict_mode: str | None = None, model_path: str | None = None):
    """Replace every QuantizedSwitchGLU with a StreamedSwitchGLU over
    ``cache`` (streaming.py:2575-2688, same arguments).  Returns the
    PrefetchRing over the streamed layers (ring.py), which also indexes and
    iterates like the list of layers.  The cache's layer keys must be the
    module paths.  ``tensor_index``/``model_path`` locate checkpoint bytes in
    the reference; here the cache's pinned host store already holds them, so
    they are accepted and unused.  ``predict_mode`` "on" / "off" pins route
    prediction (config.PREDICT_DEPTH layers ahead); "auto" lets the ring's A/B
    governor decide from measured tokens/s (None: config.PREDICT, default
    auto).  ``prefetch_depth`` > 0 turns on the previous-token heuristic.  Speculation
    only reads into free slots, so it never changes an output."""
    if predict_mode not in (None, "off", "auto", "on"):
        raise ValueError(f"predict_mode={predict_mode!r}: expected off, auto or on")
    del tensor_index, model_path
    glus = find_switch_glus(model)
    if not glus:
        raise ValueError("no QuantizedSwitchGLU modules found - this model has no MoE layers")
    streamed = [StreamedSwitchGLU(path, module, cache) for path, module in glus]
    for (path, _), s in zip(glus, streamed):
        _swap_module(model, path, s)
    for (path, _), s in zip(glus, streamed):
        parent_path = path.rpartition(".")[0]
        parent = model.get_submodule(parent_path) if parent_path else None
        s.pred = parent if isinstance(parent, _MoEBlock) else None
    ring = PrefetchRing(streamed, cache)
    if predict_mode is not None:
        ring.governor.set_mode(predict_mode)
    if prefetch_depth:
        ring.prefetch_depth = int(prefetch_depth)
    model._pagedmoe_cache = cache
    model._pagedmoe_ring = ring
    if cache.n_experts * len(glus) <= cache.routed_slots:
        cache.load_stitch()
    return ring


def get_stats(model: nn.Module) -> dict:
    """Residency counters of a patched model (loader.py:1003)."""
    K.check_workspace_errors()
    cache = getattr(model, "_pagedmoe_cache", None)
    if cache is None:
        return {}
    out = {"cache": cache.stats()}
    ring = getattr(model, "_pagedmoe_ring", None)
    if ring is not None:
        out["ring"] = ring.stats()
    return out
