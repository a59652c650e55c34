"""The streamed MoE layers of one model, in order, and their per-token state.

Counterpart of the reference's PrefetchRing (streaming.py:1404-2299), which
patch_model returns.  It carries speculative prefetch and flow decode (a
decode token whose MoE layers never wait on the host, streaming.py:675-749,
cache.py:791-910).

Speculative prefetch (route prediction, streaming.py:2013-2299).  After a
decode layer L has enqueued its compute, the routers of layers L+2 ..
L+1+PREDICT_DEPTH (on a stride of PREDICT_DEPTH layers, so each layer is
predicted once) run on layer L's last-token hidden state, their top-k +
PREDICT_SLACK ids are chosen on the GPU (the same routing kernels as the
demand path), and the ids ride layer L+1's routing sync to the host -- no
sync of their own.  After layer L+1's fetch and compute are enqueued, the
guesses are issued as speculative reads into free slots
(ExpertCache.speculate: a separate copy engine, never an eviction), so they
run under the compute of the layers between; the target layer's fetch
claims the ones it routes.  Precision is counted the reference's way:
predicted ids issued and used at the target's demand (pred_issued,
pred_used).  The targets start two layers out because the ids reach the host
one layer later (streaming.py:2002).  PREFETCH_DEPTH adds the previous-token
heuristic: the next layers' last routed ids (streaming.py:2283-2299).

Whether prediction pays is measured, not modelled (streaming.py:1790-1970):
with predict mode "auto", governor.PredictGovernor compares adjacent
windows of decode tokens run with prediction on and off.  Wrong guesses
cost copy bandwidth, so on a link-bound workload with guesses that are
often wrong it settles on off.

Flow decode.  The slot table is already on the GPU and the expert kernels
read it directly, computing an exact zero row for every routed expert that
is not resident -- the seam's contract for a dropped slot
(streaming.py:715-719) -- so a layer needs no host round trip at all.  What
the host still has to do is residency, once per token instead of once per
layer (``begin_token``, the reference's flow_pump, streaming.py:706-711):

1. wait for the previous token's kernels (one fence per token; nothing still
   queued may read a slot about to be overwritten);
2. install the admitted experts whose copies have landed (the compute stream
   is made to wait on their copy events, so no stale line survives);
3. admit the previous token's routing of every layer (cache.py:861-910):
   resident ids get recency and reuse credit, misses take a slot, possibly
   evicting, and are copied in behind the fence -- they become usable in a
   later token, never in the middle of one;
4. republish every changed table row on the compute stream.

The token's layers then run with no host sync; a routed expert that is not
resident contributes nothing to that token (the reference's flow graph omits
it the same way, streaming.py:700-702).  Tokens of more than
``config.DECODE_MAX_TOKENS`` rows (prefill) drop flow state and take the
ordinary path, and after a prefill ``config.FLOW_WARMUP`` tokens plus a hit
rate of ``config.FLOW_WARM_HIT`` are required before flow resumes
(config.py:1218-1237).  Because nothing in a flow token syncs, a token's
layers can be captured in one HIP graph and replayed after each
``begin_token``.
"""

from __future__ import annotations

import torch

from . import config
from .governor import PredictGovernor


class PrefetchRing:
    """Sequence of the model's StreamedSwitchGLU layers (iterable and
    indexable like the list patch_model used to return) plus flow state."""

    def __init__(self, layers, cache):
        self.layers = list(layers)
        self.cache = cache
        for i, layer in enumerate(self.layers):
            layer.ring = self
            layer.ring_index = i
        self.flow = bool(config.FLOW)
        self.auto_pump = True          # layer 0 calls begin_token itself
        self.token_flow = False        # the current token runs as a flow token
        self._routes: dict = {}        # layer index -> routing of the last flow token
        self._noted = False            # _routes hold a token not admitted yet
        self._pending: list = []       # admitted copy batches not installed yet
        self._fence = torch.cuda.Event()
        self._fenced = False
        self._since_prefill = 0
        self._hit_ema = 0.0
        self._miss_ema = None          # routed experts missing per token (all layers)
        self._flow_backoff = False     # flow left because the table stopped holding the routing
        self._token_stats = None
        self.flow_tokens = 0
        self.sync_tokens = 0
        # speculative prefetch
        self.predict_depth = int(config.PREDICT_DEPTH)
        self.prefetch_depth = int(config.PREFETCH_DEPTH)
        self.slack = int(config.PREDICT_SLACK)
        self._pred_gpu: list = []      # [(target index, device ids)] not yet on the host
        self._pred_host: list = []     # [(target index, ids)] waiting to be issued
        self.predicted: dict = {}      # target index -> ids guessed for its next fetch
        self.pred_issued = 0
        self.pred_used = 0
        self.spec_reads = 0
        self.governor = PredictGovernor(self, str(config.PREDICT))
        # prefill-time prediction (cache.py:2580-2650): the next layer's
        # router on this layer's MoE input, its reads started behind demand
        self._ahead_gpu = None         # (target index, device ids [N, k])
        self._ahead_host = None        # (target index, ids by predicted rows, desc)
        self._ahead_open = {}          # target index -> (reads started, claims before)
        # closed stitch (closed.py): a decode token run as one pass over the
        # live tables, kept only when no routed expert was missing
        self.closed_live = False       # closed.install ran for this model
        self.closed_armed = False      # warm enough to attempt closed tokens
        self.closed_active = False     # the current token is a closed attempt
        self.warm_streak = 0           # per-layer decode tokens in a row with no miss
        self.closed_cooldown = 0       # tokens to sit out after a replay
        self.closed_ok = 0
        self.closed_replay = 0
        self._missing = None           # device int32 [1]: missing routed experts

    # ---- sequence protocol over the layers
    def __len__(self):
        return len(self.layers)

    def __iter__(self):
        return iter(self.layers)

    def __getitem__(self, i):
        return self.layers[i]

    # ---- token boundaries
    def _flow_ready(self) -> bool:
        """Whether the next token runs as a flow token.  In flow, stay while
        the missing routed experts per token (EMA over every layer, the
        reference's critical misses, streaming.py:1585-1613) stay at or
        under FLOW_MAX_CRIT: above it the table has stopped holding what the
        router wants, and flow would be dropping experts the per-layer path
        waits for.  Out of flow, enter after FLOW_WARMUP tokens once the hit
        EMA reaches FLOW_WARM_HIT, and after such an exit only once the
        misses are back under half the bar."""
        if not self.flow:
            return False
        bar = float(config.FLOW_MAX_CRIT)
        miss = self._miss_ema
        if self.token_flow:
            if bar > 0 and miss is not None and miss > bar:
                self._flow_backoff = True
                return False
            return True
        if self._since_prefill < int(config.FLOW_WARMUP) or self._hit_ema < float(config.FLOW_WARM_HIT):
            return False
        if bar > 0 and self._flow_backoff and miss is not None and miss > bar / 2:
            return False
        return True

    def layer_call(self, index: int, n_tokens: int):
        """Called by each layer on entry: "closed" inside a closed-stitch
        attempt, "flow" when this call runs as part of a flow token, else
        None (the per-layer path).  Layer 0 opens the token."""
        if self.closed_active and n_tokens <= config.DECODE_MAX_TOKENS:
            return "closed"
        if n_tokens > config.DECODE_MAX_TOKENS:
            if index == 0:
                self.flow_drop()
                self.token_flow = False
                self._since_prefill = 0
                self._hit_ema = 0.0
            return None
        if index == 0:
            self._close_token_stats()
            was_flow, self.token_flow = self.token_flow, self._flow_ready()
            if was_flow and not self.token_flow:
                self.flow_drop()           # land and install what flow admitted
            if self.token_flow and self.auto_pump:
                self.begin_token()
            self._since_prefill += 1
            if not self.token_flow:
                self.governor.token()
            st = self.cache.raw_stats()
            self._token_stats = (st.hits, st.misses)
            if self.token_flow:
                self.flow_tokens += 1
            else:
                self.sync_tokens += 1
        return "flow" if self.token_flow else None

    # ---- closed stitch
    def begin_closed(self) -> None:
        """Open a closed-stitch attempt: every changed table row is
        republished (the attempt reads the live residency), and the device
        miss counter is zeroed with a fill kernel (no memset, so the token
        may be captured)."""
        c = self.cache
        for layer in self.layers:
            c.sync_table(layer.layer_key)
        if self._missing is None:
            self._missing = torch.zeros(1, dtype=torch.int32, device=c.slab.buf.device)
        else:
            self._missing.zero_()
        self.closed_active = True

    def count_missing(self, table, ids) -> None:
        """Add the layer's routed experts that ``table`` does not hold to the
        attempt's device counter (no sync)."""
        from . import kernels as K
        K.count_missing(table, ids.reshape(-1).contiguous(), self.cache.n_experts, self._missing)

    def end_closed(self) -> int:
        """Close the attempt; the one host read of a closed token: the number
        of routed experts that were not resident."""
        self.closed_active = False
        return int(self._missing.item())

    def _close_token_stats(self):
        if self._token_stats is None:
            return
        st = self.cache.raw_stats()
        h, m = st.hits - self._token_stats[0], st.misses - self._token_stats[1]
        if h + m:
            self._hit_ema = 0.5 * self._hit_ema + 0.5 * (h / (h + m))
            self._miss_ema = m if self._miss_ema is None else 0.7 * self._miss_ema + 0.3 * m
        self._token_stats = None

    def begin_token(self, replayed: bool = False) -> None:
        """flow_pump: fence, install landed copies, admit the last token's
        routing, republish changed rows.  With ``auto_pump`` False (a token
        captured in a graph) the caller runs this before each token, with
        ``replayed`` True once a replay of the captured token has run (the
        routing tensors noted during capture then hold that replay's ids).
        Copies into evicted slots are fenced on the compute stream's tail, so
        the host fence is not needed for safety, only to read the routing."""
        c = self.cache
        if self._fenced:
            self._fence.synchronize()
            self._fenced = False
        c.drop_staged()                  # flow tokens claim no guesses
        self._pending = c.flow_install_ready(self._pending)
        batch = []
        if self._noted or replayed:
            for i in sorted(self._routes):
                ids = sorted({int(e) for e in self._routes[i].reshape(-1).tolist()
                              if 0 <= int(e) < c.n_experts})
                batch.append((self.layers[i].layer_key, ids))
        self._noted = False
        if batch:
            fb = c.flow_admit(batch)
            if fb is not None:
                self._pending.append(fb)
        for layer in self.layers:
            c.sync_table(layer.layer_key)

    def note(self, index: int, inds: torch.Tensor) -> None:
        """A flow layer's routing (device tensor, read at the next
        begin_token); the last layer fences the token.  Under graph capture
        the tensor is the graph's own output, refreshed by every replay."""
        self._routes[index] = inds
        if torch.cuda.is_current_stream_capturing():
            return
        self._noted = True
        if index == len(self.layers) - 1:
            self._fence.record()
            self._fenced = True

    # ---- speculative prefetch
    def _router_of(self, index):
        blk = getattr(self.layers[index], "pred", None)
        return blk if blk is not None and hasattr(blk, "predict_ids") else None

    def predict(self, index: int, x2: torch.Tensor) -> None:
        """Enqueue the route prediction of the layers this stride covers on
        the last token's hidden state (device ids; no sync)."""
        d = self.predict_depth
        if d <= 0 or index % d != 0:
            return
        x_last = x2[-1:]
        for tgt in range(index + 2, index + 2 + d):
            if tgt >= len(self.layers):
                break
            blk = self._router_of(tgt)
            if blk is not None:
                self._pred_gpu.append((tgt, blk.predict_ids(x_last, self.slack)))

    def collect_predictions(self) -> None:
        """After a routing sync: the pending predictions are complete; bring
        their ids to the host (a small copy, no extra wait)."""
        for tgt, ids in self._pred_gpu:
            self._pred_host.append((tgt, sorted({int(e) for e in ids.reshape(-1).tolist()})))
        self._pred_gpu = []
        if self._ahead_gpu is not None:
            tgt, ids = self._ahead_gpu
            self._ahead_gpu = None
            counts = torch.bincount(ids.reshape(-1).long().clamp_min(0),
                                    minlength=self.cache.n_experts).cpu()
            order = sorted(range(len(counts)), key=lambda e: (-int(counts[e]), e))
            self._ahead_host = (tgt, [e for e in order if counts[e] > 0])

    # ---- prefill-time prediction
    def predict_prefill(self, index: int, x2: torch.Tensor) -> None:
        """Before layer ``index``'s routed-id sync in a prefill call: route
        the call's rows through the next layer's router (device ids; they
        ride that sync to the host)."""
        self._ahead_gpu = self._ahead_host = None
        if not config.PREFILL_AHEAD or x2 is None or index + 1 >= len(self.layers):
            return
        blk = self._router_of(index + 1)
        if blk is not None and not self.cache.stitched:
            self._ahead_gpu = (index + 1, blk.predict_ids(x2, 0))

    def issue_prefill_ahead(self, index: int) -> int:
        """Layer ``index``'s own reads are all queued: start the predicted
        reads of the next layer, behind a fence at the stream's tail.
        Returns the reads started."""
        if self._ahead_host is None or self._ahead_host[0] != index + 1:
            return 0
        tgt, ids = self._ahead_host
        self._ahead_host = None
        c = self.cache
        c.spec_fence()
        before = c.raw_stats().ahead_claims
        n = c.prefill_ahead(self.layers[tgt].layer_key, ids)
        if n:
            self._ahead_open[tgt] = (n, before)
        return n

    def settle_prefill_ahead(self, index: int) -> None:
        """Layer ``index``'s prefill groups are done: score its guesses."""
        got = self._ahead_open.pop(index, None)
        if got is not None:
            n, before = got
            self.cache.note_ahead(n, self.cache.raw_stats().ahead_claims - before)

    def note_demand(self, index: int, ids) -> None:
        """A layer's fetch: score its prediction (pred_issued / pred_used)."""
        guess = self.predicted.pop(index, None)
        if guess:
            self.pred_issued += len(guess)
            self.pred_used += len(guess & set(int(e) for e in ids))

    def speculate(self, index: int, x2: torch.Tensor) -> None:
        """After layer ``index`` enqueued its compute: issue the collected
        guesses for layers still ahead, the previous-token heuristic, and
        the next prediction."""
        c = self.cache
        if c.stitched or self.token_flow:
            return
        ready, self._pred_host = self._pred_host, []
        for tgt, ids in ready:
            if tgt > index:
                self.predicted.setdefault(tgt, set()).update(ids)
                self.spec_reads += c.speculate(self.layers[tgt].layer_key, ids)
        for d in range(1, self.prefetch_depth + 1):
            nxt = self.layers[(index + d) % len(self.layers)]
            if nxt.last_ids:
                self.spec_reads += c.speculate(nxt.layer_key, nxt.last_ids)
        self.predict(index, x2)

    def flow_drop(self) -> None:
        """Leave flow: wait for and install every admitted copy, forget the
        last token's routing (a prefill replaces it)."""
        if self._fenced:
            self._fence.synchronize()
            self._fenced = False
        self._pending = self.cache.flow_install_ready(self._pending, wait=True)
        self._routes.clear()
        self._noted = False
        self._pred_gpu, self._pred_host = [], []
        self.predicted.clear()
        self.cache.drop_staged()
        for layer in self.layers:
            self.cache.sync_table(layer.layer_key)

    def stats(self) -> dict:
        return {"flow": self.flow, "flow_tokens": self.flow_tokens,
                "closed_armed": self.closed_armed, "closed_ok": self.closed_ok,
                "closed_replay": self.closed_replay,
                "predict": self.governor.describe(),
                "sync_tokens": self.sync_tokens, "pending_batches": len(self._pending),
                "hit_ema": self._hit_ema, "miss_ema": self._miss_ema,
                "predict_depth": self.predict_depth,
                "pred_issued": self.pred_issued, "pred_used": self.pred_used,
                "pred_precision": self.pred_used / self.pred_issued if self.pred_issued else None,
                "spec_reads": self.spec_reads}
