"""CPU oracle for the routed-expert MoE hot path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker.  The product path
(``pagedmoe_amd``) never imports it and fails loudly without its HIP library.

The reference (noahclark556/paged-moe) keeps the arithmetic of this path in
its un-vendored dependencies (mlx==0.32.2, mlx-lm==0.31.3), which are absent
here.  This module restates the behaviour from the reference's own call sites,
tests and probes (cited per function) and fixes every choice the reference
leaves open so that the HIP kernels can be held to it bit for bit:

* router logits: fp32, a *canonical* summation order (64 lane partials over
  16-byte chunks, then an xor butterfly) -- exactly the order the HIP router
  kernel uses, so logits and therefore routing indices are bit-exact;
* exp/sigmoid: ``pexp``, Cody-Waite argument reduction plus a degree-7 Taylor
  polynomial evaluated with separately rounded mul/add (no fma), so numpy, C
  and the GPU all produce the same bits;
* top-k ties: higher value first, lower expert id wins a tie; output sorted;
* affine g64 format: little-endian bit stream per row, ``w = s*q + b``;
* dispatch: ``numpy.argsort(kind="stable")`` of the flat ids (the reference's
  own closed form, streaming.py:794).

Pinning status of each function is recorded in ``PINNING`` below; a function
that none of the independent checks in ``tests/test_oracle.py`` pins is marked
"parity unpinned" there.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np

# -- which independent check pins each oracle function (tests/test_oracle.py)
PINNING = {
    "bf16_round": "closed form vs float64 midpoint rule; torch.bfloat16 cast",
    "router_logits": "float64 exact dot within fp32 error bound; brute force lane order on tiny D",
    "pexp": "float64 exp within 2 ulp over a dense grid; exp(0)=1, exp(ln2)=2",
    "softmax_topk": "brute-force full sort; K=E special case; sums to 1; "
                    "top-k(logits)==top-k(softmax) (streaming.py:2068-2073); "
                    "float64 softmax; reference test_stream.py:191-196 restated by torch",
    "sigmoid_group_topk": "brute-force enumeration of all group subsets on tiny E; "
                          "n_group=1 reduces to plain top-k; scores sum to routed scale; "
                          "_unit_mass KAT (test_moe_gate_routing.py:28-34)",
    "dispatch": "np.argsort stable closed form (streaming.py:794); permutation, "
                "sortedness, tie order and bincount invariants; brute force",
    "quant_pack": "bit-layout KAT (values 0..7 -> 0x76543210); pack/unpack round trip; "
                  "6-bit 3-byte-pack closed form; |dequant(quant(w))-w| <= s/2",
    "dequant": "closed form s*q+b (safetensors_index layout); torch bf16 cast",
    "expert_ffn": "torch float64 dense reference (F.silu, matmul) on dequantized weights",
    "combine": "closed form (test_stream.py:198) vs float64 einsum",
    "slot_policy": "reference KATs: full stitch set unevictable (test_stitch.py:53-58), "
                   "admit installs+MRU+hit count (test_flow.py:88-118), every slot "
                   "accounted once (test_prefill_slab.py:79-99); brute-force LRU on "
                   "tiny traces with LFRU off; hand-worked traces from the text of "
                   "cache.py (tests/slot_kats.py): the LFRU second chance, plain LRU, "
                   "pins over budget, prefill after a warm decode and into a cold slab, "
                   "flow admission, speculation (claims, hand-back) and prefill-time "
                   "prediction (floors, free then stage slots, claims); an independent "
                   "list-plus-counter LFRU over Zipf traces",
    "unit_mass": "KAT test_moe_gate_routing.py:28-34",
}

LANES = 64          # wavefront width; router partial sums per output
CHUNK = 8           # bf16 elements per 16-byte load
SPAN = LANES * CHUNK  # 512 elements per pass of a wave over a row


# ---------------------------------------------------------------- bf16

def bf16_round(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = 0x7FC0
    return r


def bf16_to_f32(b) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- exp

_LOG2E = np.float32(1.44269504)
_C1 = np.float32(0.693359375)        # ln2 high part, 9 significant bits
_C2 = np.float32(-2.12194440e-4)     # ln2 - C1
_TAYLOR = [np.float32(1.0 / 5040.0), np.float32(1.0 / 720.0),
           np.float32(1.0 / 120.0), np.float32(1.0 / 24.0),
           np.float32(1.0 / 6.0), np.float32(0.5), np.float32(1.0),
           np.float32(1.0)]
EXP_LO = np.float32(-86.0)           # below: result is 0 (no subnormals)


def pexp(x) -> np.ndarray:
    """exp(x) in float32 with only separately rounded +,-,*, rint and ldexp.

    Cody & Waite (1980) reduction x = n*ln2 + r with ln2 split in two, then the
    Taylor series of e^r to degree 7 in Horner form.  |r| <= 0.35 so the
    truncation error is below 0.1 ulp.  Bit-identical in numpy, C
    (-ffp-contract=off) and the HIP kernels.
    """
    x = np.asarray(x, dtype=np.float32)
    n = np.rint(x * _LOG2E).astype(np.float32)
    r = x - n * _C1
    r = r - n * _C2
    p = _TAYLOR[0]
    for c in _TAYLOR[1:]:
        p = p * r + c
    p = np.asarray(p, dtype=np.float32)
    n_c = np.clip(n, -200, 200).astype(np.int32)
    with np.errstate(over="ignore"):
        out = np.ldexp(p, n_c).astype(np.float32)
    out = np.where(x < EXP_LO, np.float32(0.0), out)
    return out.astype(np.float32)


def psigmoid(x) -> np.ndarray:
    """1 / (1 + pexp(-x)), correctly rounded division."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", divide="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + pexp(-x))).astype(np.float32)


# ---------------------------------------------------------------- router

def router_logits(x_bits, w_bits, logit_bias=None) -> np.ndarray:
    """Router logits L = x . Wg^T in float32, canonical order.

    Restates the router ``nn.Linear`` the reference taps (streaming.py:167-193,
    re-read :431-443; the block call ``self.gate(x)`` in mlx-lm).  Canonical
    order, shared with the HIP kernel: element d = 512*t + 8*l + j goes to
    lane l; each lane accumulates fma(x_d, w_d, acc) for t ascending, j
    ascending (bf16*bf16 is exact in fp32, so ``acc + x*w`` here is that fma);
    the 64 lane partials are then combined by an xor butterfly with strides
    32,16,8,4,2,1.  ``logit_bias`` (float32 [E]) is added after the sum; it is
    the per-expert skew of the uneven-load prefill workload.
    """
    x = bf16_to_f32(x_bits)
    w = bf16_to_f32(w_bits)
    n, d = x.shape
    e = w.shape[0]
    assert w.shape[1] == d and d % CHUNK == 0
    t_n = -(-d // SPAN)
    pad = t_n * SPAN - d
    if pad:
        x = np.concatenate([x, np.zeros((n, pad), np.float32)], axis=1)
        w = np.concatenate([w, np.zeros((e, pad), np.float32)], axis=1)
    x = x.reshape(n, t_n, LANES, CHUNK)
    w = w.reshape(e, t_n, LANES, CHUNK)
    acc = np.zeros((n, e, LANES), np.float32)
    for t in range(t_n):
        for j in range(CHUNK):
            acc += x[:, None, t, :, j] * w[None, :, t, :, j]
    acc = butterfly(acc)
    out = acc[..., 0]
    if logit_bias is not None:
        out = out + np.asarray(logit_bias, np.float32)[None, :]
    return out.astype(np.float32)


def butterfly(acc: np.ndarray) -> np.ndarray:
    """xor butterfly over the last axis (64 lanes); every lane ends equal."""
    lanes = np.arange(acc.shape[-1])
    off = acc.shape[-1] // 2
    while off:
        acc = acc + acc[..., lanes ^ off]
        off //= 2
    return acc


def lane_sum(v: np.ndarray) -> np.ndarray:
    """Canonical sum of the last axis: element i -> lane i % 64 (sequential
    per lane in ascending i), then butterfly.  Used for the full-softmax
    denominator over E experts."""
    n = v.shape[-1]
    rows = -(-n // LANES)
    pad = rows * LANES - n
    if pad:
        v = np.concatenate([v, np.zeros(v.shape[:-1] + (pad,), np.float32)], axis=-1)
    v = v.reshape(v.shape[:-1] + (rows, LANES))
    acc = np.zeros(v.shape[:-2] + (LANES,), np.float32)
    for i in range(rows):
        acc = acc + v[..., i, :]
    return butterfly(acc)[..., 0]


def topk_desc(vals: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest per row, sorted descending; ties -> lower id."""
    order = np.argsort(-vals, axis=-1, kind="stable")
    return order[..., :k].astype(np.int32)


def softmax_topk(logits, k: int, norm_topk_prob: bool = True):
    """Qwen3-MoE / Qwen3-Next routing.

    Reference: the block restated at tests/test_stream.py:191-196
    (softmax(precise) -> argpartition top-k -> take -> renorm) and the weight
    re-derivation ``mx.softmax(sel)`` at streaming.py:2443-2452.  Selection is
    by logit (softmax is monotone), ties to the lower expert id, slots sorted
    by descending weight.  With ``norm_topk_prob`` the weights are the softmax
    over the selected logits; without it, the selected entries of the full
    softmax (denominator summed in canonical lane order).
    """
    logits = np.asarray(logits, np.float32)
    inds = topk_desc(logits, k)
    sel = np.take_along_axis(logits, inds, axis=-1)
    m = sel[..., :1]
    ex = pexp(sel - m)
    if norm_topk_prob:
        s = np.zeros(ex.shape[:-1], np.float32)
        for j in range(k):
            s = s + ex[..., j]
    else:
        s = lane_sum(pexp(logits - m))
    w = (ex / s[..., None]).astype(np.float32)
    return inds, w


def sigmoid_group_topk(logits, bias, n_group: int, topk_group: int, k: int,
                       norm_topk_prob: bool = True, routed_scale: float = 1.0):
    """DeepSeek-V3 / Kimi-K2 ``noaux_tc`` routing (mlx-lm deepseek_v3.MoEGate).

    The reference consumes the gate's (inds, scores) at streaming.py:2424-2442;
    config fields at tests/test_dsa_shared.py:27-45.  sigma = sigmoid(L);
    c = sigma + bias; group score = sum of the two largest c in the group;
    keep ``topk_group`` groups (ties -> lower group id); c of other groups is
    masked to 0.0; top-k by masked c (ties -> lower id); weight = sigma of the
    pick, normalised to sum 1 over the picks when ``norm_topk_prob``, then times
    ``routed_scale``.
    """
    logits = np.asarray(logits, np.float32)
    n, e = logits.shape
    sig = psigmoid(logits)
    c = (sig + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    if n_group > 1:
        gs = e // n_group
        cg = c.reshape(n, n_group, gs)
        top2 = -np.sort(-cg, axis=-1)[..., :2]
        gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)
        keep = topk_desc(gscore, topk_group)
        mask = np.zeros((n, n_group), bool)
        np.put_along_axis(mask, keep, True, axis=-1)
        c = np.where(np.repeat(mask, gs, axis=-1), c, np.float32(0.0))
    inds = topk_desc(c, k)
    w = np.take_along_axis(sig, inds, axis=-1).astype(np.float32)
    if norm_topk_prob:
        s = np.zeros((n,), np.float32)
        for j in range(k):
            s = s + w[:, j]
        w = (w / s[:, None]).astype(np.float32)
    w = (w * np.float32(routed_scale)).astype(np.float32)
    return inds, w


def unit_mass(w) -> np.ndarray:
    """Rows rescaled to sum 1 (streaming.py:2326-2335)."""
    w = np.asarray(w, np.float32)
    return w / np.maximum(w.sum(axis=-1, keepdims=True), 1e-6)


# ---------------------------------------------------------------- dispatch

@dataclass
class Dispatch:
    order: np.ndarray    # [N*K] int32: flat (token,k) positions grouped by expert
    counts: np.ndarray   # [E] int32
    offsets: np.ndarray  # [E+1] int32, exclusive scan of counts
    inv: np.ndarray      # [N*K] int32: inv[order[i]] = i
    active: np.ndarray   # ascending expert ids with counts > 0


def dispatch(inds, n_experts: int) -> Dispatch:
    """Stable token->expert dispatch (streaming.py:789-801, :833-836;
    bench/prefill_gather_probe.py:52-55)."""
    flat = np.asarray(inds).reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size, dtype=np.int32)
    active = np.nonzero(counts)[0].astype(np.int32)
    return Dispatch(order, counts, offsets, inv, active)


# ---------------------------------------------------------------- quant format

def words_per_row(cols: int, bits: int) -> int:
    assert (cols * bits) % 32 == 0
    return cols * bits // 32


def pack_rows(q: np.ndarray, bits: int) -> np.ndarray:
    """[R, C] integers < 2^bits -> [R, C*bits/32] uint32, little-endian bit
    stream per row (value i occupies stream bits [i*bits, i*bits+bits))."""
    q = np.asarray(q, np.uint64)
    r, c = q.shape
    nw = words_per_row(c, bits)
    out = np.zeros((r, nw + 1), np.uint64)
    pos = np.arange(c, dtype=np.uint64) * np.uint64(bits)
    word = (pos // np.uint64(32)).astype(np.int64)
    sh = pos % np.uint64(32)
    v = q << sh[None, :]
    lo = v & np.uint64(0xFFFFFFFF)
    hi = v >> np.uint64(32)
    for col in range(c):
        out[:, word[col]] |= lo[:, col]
        out[:, word[col] + 1] |= hi[:, col]
    return out[:, :nw].astype(np.uint32)


def unpack_rows(w: np.ndarray, bits: int, cols: int) -> np.ndarray:
    """Inverse of ``pack_rows``: [R, C*bits/32] uint32 -> [R, C] uint8."""
    w = np.asarray(w, np.uint64)
    r = w.shape[0]
    ext = np.concatenate([w, np.zeros((r, 1), np.uint64)], axis=1)
    pos = np.arange(cols, dtype=np.uint64) * np.uint64(bits)
    word = (pos // np.uint64(32)).astype(np.int64)
    sh = pos % np.uint64(32)
    v = (ext[:, word] | (ext[:, word + 1] << np.uint64(32))) >> sh[None, :]
    return (v & np.uint64((1 << bits) - 1)).astype(np.uint8)


@dataclass
class QTensor:
    """One affine-quantized projection: weight [O, I*b/32] u32, scales and
    biases bf16 bits [O, I/g] (safetensors_index.py:8-25; slab.py:82-126)."""
    weight: np.ndarray
    scales: np.ndarray
    biases: np.ndarray
    bits: int
    group: int
    cols: int

    @property
    def rows(self) -> int:
        return self.weight.shape[0]


def quantize(w, bits: int, group: int = 64) -> QTensor:
    """Min/max affine quantizer used to build every fixture and synthetic
    weight.  Per group: scale = (max-min)/(2^b-1) and bias = min, both stored
    as bf16 (a zero scale becomes 1.0); q = clip(rint((w - bias)/scale)) with
    the *stored* bf16 values.  mlx's own quantizer variant is unpinned here;
    this one is the format of record for the fixtures."""
    w = np.asarray(w, np.float32)
    o, i = w.shape
    assert i % group == 0
    g = i // group
    wg = w.reshape(o, g, group)
    lo = wg.min(axis=-1)
    hi = wg.max(axis=-1)
    scale = ((hi - lo) / np.float32((1 << bits) - 1)).astype(np.float32)
    s_bits = bf16_round(scale)
    b_bits = bf16_round(lo)
    s = bf16_to_f32(s_bits)
    s_bits = np.where(s == 0, np.uint16(0x3F80), s_bits).astype(np.uint16)
    s = bf16_to_f32(s_bits)
    b = bf16_to_f32(b_bits)
    with np.errstate(invalid="ignore"):
        q = np.rint((wg - b[..., None]) / s[..., None])
    q = np.clip(np.nan_to_num(q), 0, (1 << bits) - 1).astype(np.uint8).reshape(o, i)
    return QTensor(pack_rows(q, bits), s_bits, b_bits, bits, group, i)


def dequant_f32(qt: QTensor) -> np.ndarray:
    """w = s*q + b in float32 (s*q is exact, so this is one rounding, the same
    as fmaf).  Closed form of mlx affine dequantization."""
    q = unpack_rows(qt.weight, qt.bits, qt.cols).astype(np.float32)
    o = qt.rows
    g = qt.cols // qt.group
    s = np.repeat(bf16_to_f32(qt.scales).reshape(o, g), qt.group, axis=1)
    b = np.repeat(bf16_to_f32(qt.biases).reshape(o, g), qt.group, axis=1)
    return (s * q + b).astype(np.float32)


def dequant_bf16(qt: QTensor) -> np.ndarray:
    """Dequantized weights as bf16 bits (round to nearest even)."""
    return bf16_round(dequant_f32(qt))


def dequant_f64(qt: QTensor) -> np.ndarray:
    q = unpack_rows(qt.weight, qt.bits, qt.cols).astype(np.float64)
    o = qt.rows
    g = qt.cols // qt.group
    s = np.repeat(bf16_to_f32(qt.scales).astype(np.float64).reshape(o, g), qt.group, axis=1)
    b = np.repeat(bf16_to_f32(qt.biases).astype(np.float64).reshape(o, g), qt.group, axis=1)
    return s * q + b


# ---------------------------------------------------------------- experts

@dataclass
class Expert:
    gate: QTensor
    up: QTensor
    down: QTensor


def make_expert(rng, hidden: int, inter: int, bits: int, group: int = 64,
                std: float = 0.02) -> Expert:
    """Expert from N(0, std) fp32 weights (gate/up [I, D], down [D, I])."""
    g = rng.standard_normal((inter, hidden), dtype=np.float32) * np.float32(std)
    u = rng.standard_normal((inter, hidden), dtype=np.float32) * np.float32(std)
    d = rng.standard_normal((hidden, inter), dtype=np.float32) * np.float32(std)
    return Expert(quantize(g, bits, group), quantize(u, bits, group),
                  quantize(d, bits, group))


def expert_ffn_f64(x_f32: np.ndarray, ex: Expert, dense=None) -> np.ndarray:
    """down(silu(gate x) * (up x)) in float64 on dequantized weights.
    SwiGLU as mlx-lm's ``SwiGLU`` / streaming.py:500 (restated
    bench/prefill_gather_probe.py:61,74 as silu(gate)*up)."""
    if dense is None:
        dense = (dequant_f64(ex.gate), dequant_f64(ex.up), dequant_f64(ex.down))
    wg, wu, wd = dense
    x = np.asarray(x_f32, np.float64)
    g = x @ wg.T
    u = x @ wu.T
    h = g / (1.0 + np.exp(-g)) * u
    return h @ wd.T


def switch_glu_f64(x_bits, inds, experts, dense_cache=None) -> np.ndarray:
    """The seam contract: y[n, k] = FFN_{inds[n,k]}(x[n]) -> [N, K, D]
    (streaming.py:946-1401 returns per-slot, uncombined rows in (token, k)
    order; _run_slab :587-631)."""
    x = bf16_to_f32(x_bits)
    n, k = inds.shape
    d = x.shape[1]
    y = np.zeros((n, k, d), np.float64)
    disp = dispatch(inds, int(np.max(inds)) + 1 if inds.size else 1)
    for e in disp.active:
        rows = disp.order[disp.offsets[e]:disp.offsets[e + 1]]
        toks = rows // k
        dense = None if dense_cache is None else dense_cache.get(int(e))
        if dense is None:
            ex = experts[int(e)]
            dense = (dequant_f64(ex.gate), dequant_f64(ex.up), dequant_f64(ex.down))
            if dense_cache is not None:
                dense_cache[int(e)] = dense
        yr = expert_ffn_f64(x[toks], experts[int(e)], dense)
        y[toks, rows % k] = yr
    return y


def combine_f64(y, w, shared=None) -> np.ndarray:
    """out[n] = sum_k w[n,k] y[n,k] (+ shared[n]); test_stream.py:198."""
    out = np.einsum("nk,nkd->nd", np.asarray(w, np.float64), np.asarray(y, np.float64))
    if shared is not None:
        out = out + shared
    return out


def combine_f32(y_f32, w, shared=None, shared_w=None) -> np.ndarray:
    """Fixed-order fp32 combine: acc = fma(w_k, y_k, acc) for k ascending,
    then acc = fma(s, shared, acc) with s = shared_w[n] (1 when None), then
    round to bf16 (bits).  This is the deterministic order of the HIP combine.
    Each fma is formed exactly in float64 (a float32 product has at most 48
    significant bits) and rounded once more to float32."""
    y = np.asarray(y_f32, np.float64)
    w = np.asarray(w, np.float64)
    acc = np.zeros((y.shape[0], y.shape[2]), np.float32)
    for j in range(y.shape[1]):
        acc = (acc.astype(np.float64) + w[:, j, None] * y[:, j, :]).astype(np.float32)
    if shared is not None:
        s = np.ones(y.shape[0]) if shared_w is None else np.asarray(shared_w, np.float64)
        acc = (acc.astype(np.float64) + s[:, None] * np.asarray(shared, np.float64)).astype(np.float32)
    return bf16_round(acc)


# ---------------------------------------------------------------- slot policy

@dataclass
class SlotPolicy:
    """Slab slot table restated from ExpertCache (cache.py:410).

    * free list ``list(range(slots-1,-1,-1))`` popped from the end, so the
      first allocation is slot 0 (cache.py:991, :1138-1139);
    * reserve ``max(4, int(slots*reserve_frac))`` slots, budget = the rest
      (cache.py:996-1002); no reserve once a full stitch set is resident;
    * a layer step clears pins, classifies ids (hit: MRU + freq=min(8,freq+1),
      pinned), then gives each miss a slot: free slot, else evict the
      least-recent unpinned non-stitch entry (cache.py:2327-2453, :1118-1159);
    * installs run in ascending expert id (the reference installs in read
      completion order, cache.py:2482-2519; this contract fixes it), each
      followed by the LFRU second-chance trim (cache.py:2236-2291).
    """
    slots: int
    reserve_frac: float = 0.1
    lfru: bool = True
    lfru_scan: int = 8
    freq_max: int = 8
    lru: "OrderedDict" = field(default_factory=OrderedDict)
    slot_of: dict = field(default_factory=dict)
    freq: dict = field(default_factory=dict)
    pinned: set = field(default_factory=set)
    stitch_keys: set = field(default_factory=set)
    hits: int = 0
    misses: int = 0
    evictions: int = 0
    starved: int = 0

    def __post_init__(self):
        self.free = list(range(self.slots - 1, -1, -1))
        self.reserve = max(4, int(self.slots * self.reserve_frac))
        self.budget = self.slots - self.reserve

    def _evict(self, key):
        self.lru.pop(key)
        self.freq.pop(key, None)
        self.evictions += 1
        slot = self.slot_of.pop(key)
        self.free.append(slot)

    def _alloc(self, evict_ok=True):
        if self.free:
            return self.free.pop()
        if not evict_ok:
            return None
        for key in list(self.lru):
            if key in self.stitch_keys or self.slot_of.get(key) in self.pinned:
                continue
            self._evict(key)
            if self.free:
                return self.free.pop()
        staged = self.__dict__.get("staged")
        if staged:  # give up an unclaimed guess, the latest first (cache.py:1149-1157)
            key = next(reversed(staged))
            return staged.pop(key)
        self.starved += 1
        return None

    def _trim(self):
        scan = self.lfru_scan if self.lfru else 0
        while len(self.lru) > self.budget and len(self.lru) > 1:
            for _ in range(scan):
                if len(self.lru) <= 1:
                    break
                key = next(iter(self.lru))
                f = self.freq.get(key, 0)
                if f <= 0:
                    break
                self.freq[key] = f >> 1
                self.lru.move_to_end(key)
            victim = None
            for key in self.lru:
                if key in self.stitch_keys or self.slot_of.get(key) in self.pinned:
                    continue
                victim = key
                break
            if victim is None:
                break
            self._evict(victim)

    def step(self, layer, ids):
        """One layer fetch.  Returns (hit ids, [(miss id, slot)]) with misses
        installed.  ``ids`` is taken as a set, visited ascending.  A staged
        guess (``speculate``) is claimed: a hit installed at its slot, no
        read (cache.py:2379-2386); the layer's unclaimed guesses are handed
        back (their slots drain to the free list at the next settle)."""
        self.pinned.clear()
        staged = self.__dict__.setdefault("staged", OrderedDict())
        ids = sorted({int(e) for e in ids})
        hits, misses, claimed = [], [], []
        for e in ids:
            key = (layer, e)
            if key in self.lru:
                self.hits += 1
                self.lru.move_to_end(key)
                self.freq[key] = min(self.freq_max, self.freq.get(key, 0) + 1)
                self.pinned.add(self.slot_of[key])
                hits.append(e)
            elif key in staged and staged[key] < self.slots:
                # a guess in a prefill stage slot is never made resident
                # there; it is a miss and handed back below
                self.hits += 1
                slot = staged.pop(key)
                self.pinned.add(slot)
                claimed.append((e, slot))
                hits.append(e)
            else:
                self.misses += 1
                misses.append(e)
        placed = []
        for e in misses:
            slot = self._alloc(True)
            if slot is None:
                continue
            self.pinned.add(slot)
            placed.append((e, slot))
        for e, slot in sorted(claimed + placed):
            key = (layer, e)
            self.slot_of[key] = slot
            self.lru[key] = slot
            self._trim()
        self._drop_staged(lambda key: key[0] == layer)
        return hits, placed

    # ---- speculation (ExpertCache.prefetch cache.py:2853 with
    # evict_ok=False; staging and claim :2379-2386)

    def speculate(self, layer, ids, max_staged):
        """Guesses in priority order into free slots only, while fewer than
        max_staged are outstanding.  Returns [(id, slot)] started."""
        self.settle()
        staged = self.__dict__.setdefault("staged", OrderedDict())
        pending = getattr(self, "pending", {})
        got = []
        for e in ids:
            key = (layer, int(e))
            if key in self.lru or key in pending or key in staged or any(k == key for k, _ in got):
                continue
            if len(staged) + len(got) >= max_staged or not self.free:
                break
            got.append((key, self.free.pop()))
        for key, slot in got:
            staged[key] = slot
        return [(key[1], slot) for key, slot in got]

    def _drop_staged(self, which):
        staged = self.__dict__.setdefault("staged", OrderedDict())
        drain = self.__dict__.setdefault("draining", [])
        for key in [k for k in staged if which(k)]:
            drain.append(staged.pop(key))

    def drop_all_staged(self):
        staged = self.__dict__.setdefault("staged", OrderedDict())
        drain = self.__dict__.setdefault("draining", [])
        while staged:
            key = next(reversed(staged))
            drain.append(staged.pop(key))
        self.settle()

    def settle(self):
        """Handed-back guesses' reads have landed: their slots are free (a
        prefill stage slot goes back to the stage)."""
        drain = self.__dict__.setdefault("draining", [])
        for slot in drain:
            (self.stage_free if slot >= self.slots else self.free).append(slot)
        drain.clear()

    def prefill_ahead(self, layer, ids, free_floor, stage_floor):
        """Prefill-time prediction (cache.py:2580-2650): ids in priority
        order, skipping resident, pending and staged ones, take a free slot
        while more than ``free_floor`` are free, else a stage slot while more
        than ``stage_floor`` are free; never an eviction; the first id that
        finds neither stops the pass.  Returns [(id, slot)] started."""
        self.settle()
        if not hasattr(self, "stage_free"):
            self.set_stage(self.slots, 0)
        staged = self.__dict__.setdefault("staged", OrderedDict())
        pending = getattr(self, "pending", {})
        got, seen = [], set()
        for e in ids:
            key = (layer, int(e))
            if key in seen or key in self.lru or key in pending or key in staged:
                continue
            seen.add(key)
            if len(self.free) > free_floor:
                slot = self.free.pop()
            elif len(self.stage_free) > stage_floor:
                slot = self.stage_free.pop()
            else:
                break
            got.append((key, slot))
        for key, slot in got:
            staged[key] = slot
        return [(key[1], slot) for key, slot in got]

    # ---- prefill fetch groups (cache.py:2347-2453 with prefill=True,
    # PREFILL_TOUCH=0, PREFILL_SLAB=1; _install(..., "soft") :2306-2312;
    # the stage of ensure_stage :1345-1390, _stage_return :1427-1440)

    def set_stage(self, first_slot: int, n_slots: int) -> None:
        self.stage_free = list(range(first_slot + n_slots - 1, first_slot - 1, -1))
        self.groups = {}

    def step_prefill(self, layer, ids):
        """One prefill group.  Hits: counted, recency/frequency untouched.
        Misses (ascending id): a free slot (never an eviction), installed at
        MRU with no reuse credit while fewer than ``budget`` entries are
        resident, else held for the group; past the free list, a stage slot;
        past both, unplaced.  Returns (ticket, [(miss id, slot)], unplaced)."""
        if not hasattr(self, "stage_free"):
            self.set_stage(self.slots, 0)
        ticket = next(t for t in range(64) if t not in self.groups)
        held = {"layer": layer, "temp": [], "free": [], "stage": [], "claimed": []}
        staged = self.__dict__.setdefault("staged", OrderedDict())
        placed, unplaced = [], 0
        for e in sorted({int(i) for i in ids}):
            key = (layer, e)
            if key in self.lru:
                self.hits += 1
                continue
            if key in staged:             # its read already started: claimed
                slot = staged.pop(key)
                self.hits += 1
                held["claimed"].append((e, slot))
                if slot < self.slots and len(self.lru) < self.budget:
                    self.slot_of[key] = slot
                    self.lru[key] = slot
                else:
                    held["temp"].append((e, slot))
                    held["free" if slot < self.slots else "stage"].append(slot)
                continue
            self.misses += 1
            if self.free:
                slot = self.free.pop()
                if len(self.lru) < self.budget:
                    self.slot_of[key] = slot
                    self.lru[key] = slot
                else:
                    held["temp"].append((e, slot))
                    held["free"].append(slot)
            elif self.stage_free:
                slot = self.stage_free.pop()
                held["temp"].append((e, slot))
                held["stage"].append(slot)
            else:
                unplaced += 1
                continue
            placed.append((e, slot))
        self.groups[ticket] = held
        self._drop_staged(lambda key: key[0] == layer)
        return ticket, placed, unplaced

    def compute_row(self, ticket, n_experts) -> np.ndarray:
        g = self.groups[ticket]
        row = self.table(g["layer"], n_experts)
        for e, slot in g["temp"]:
            row[e] = slot
        return row

    def prefill_done(self, ticket) -> None:
        g = self.groups.pop(ticket)
        self.free.extend(g["free"])
        self.stage_free.extend(g["stage"])

    # ---- flow decode (flow_admit, cache.py:861-910; install on arrival,
    # _attach_staging(install_now=True) :2866-2910)

    def admit(self, layer, ids, clear_pins=True):
        """Resident ids: MRU + reuse credit.  Others: a miss; unless already
        pending, a slot (evicting) and pending until ``install``.  Stops at the
        first miss that finds no slot.  Returns [(miss id, slot)]."""
        if not hasattr(self, "pending"):
            self.pending = {}
        if clear_pins:
            self.pinned.clear()
        placed = []
        for e in sorted({int(i) for i in ids}):
            key = (layer, e)
            if key in self.lru:
                self.hits += 1
                self.lru.move_to_end(key)
                self.freq[key] = min(self.freq_max, self.freq.get(key, 0) + 1)
                continue
            self.misses += 1
            if key in self.pending:
                continue
            slot = self._alloc(True)
            if slot is None:
                break
            self.pending[key] = slot
            placed.append((e, slot))
        return placed

    def install(self, layer, ids):
        for e in sorted({int(i) for i in ids}):
            key = (layer, e)
            slot = self.pending.pop(key)
            self.slot_of[key] = slot
            self.lru[key] = slot
            self._trim()

    def stitch(self, layers, n_experts) -> bool:
        """Load every expert into a fixed slot: slot = layer_idx*E + e
        (cache.py:717-787 with the free list above)."""
        if len(layers) * n_experts > self.slots:
            return False
        for layer in layers:
            for e in range(n_experts):
                slot = self._alloc(False)
                key = (layer, e)
                self.slot_of[key] = slot
                self.lru[key] = slot
                self.stitch_keys.add(key)
        self.budget = self.slots
        return True

    def table(self, layer, n_experts) -> np.ndarray:
        """expert -> slot for installed entries, -1 otherwise
        (cache.py:791-859, flow table)."""
        t = np.full(n_experts, -1, np.int32)
        for (lk, e), slot in self.lru.items():
            if lk == layer and e < n_experts:
                t[e] = slot
        return t


# ---------------------------------------------------------------- workloads

@dataclass
class LayerSpec:
    hidden: int
    experts: int
    inter: int
    top_k: int
    bits: int = 4
    group: int = 64
    scoring: str = "softmax"        # "softmax" | "sigmoid"
    norm_topk_prob: bool = True
    n_group: int = 1
    topk_group: int = 1
    routed_scale: float = 1.0
    shared: int = 0                 # shared experts (always on)
    shared_gate: bool = False       # Qwen3-Next: sigmoid(x . g) * shared(x)


def make_layer(spec: LayerSpec, seed: int = 0, expert_ids=None):
    """Seeded synthetic layer: router weight bf16 N(0, 0.02), experts
    quantized from N(0, 0.02).  Returns (gate_w_bits [E, D], experts list,
    score bias or None, shared experts list, shared gate bits or None).
    Each part draws from its own seed sequence ending in a nonzero tag
    (numpy's SeedSequence ignores trailing zeros), so no weight is correlated
    with activations drawn from default_rng(seed)."""
    rng = np.random.default_rng([seed, 7001])
    gw = bf16_round(rng.standard_normal((spec.experts, spec.hidden), dtype=np.float32)
                    * np.float32(0.02))
    ids = range(spec.experts) if expert_ids is None else expert_ids
    experts = {}
    for e in range(spec.experts):
        sub = np.random.default_rng([seed, e, 7002])
        if e in ids:
            experts[e] = make_expert(sub, spec.hidden, spec.inter, spec.bits, spec.group)
    bias = None
    if spec.scoring == "sigmoid":
        bias = (rng.standard_normal(spec.experts, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    shared = [make_expert(np.random.default_rng([seed, s, 7003]), spec.hidden, spec.inter,
                          spec.bits, spec.group) for s in range(spec.shared)]
    sg = None
    if spec.shared_gate:
        sg = bf16_round(rng.standard_normal((1, spec.hidden), dtype=np.float32) * np.float32(0.02))
    return gw, experts, bias, shared, sg


def route(spec: LayerSpec, logits, bias=None):
    if spec.scoring == "softmax":
        return softmax_topk(logits, spec.top_k, spec.norm_topk_prob)
    return sigmoid_group_topk(logits, bias, spec.n_group, spec.topk_group, spec.top_k,
                              spec.norm_topk_prob, spec.routed_scale)


def moe_layer_f64(spec: LayerSpec, x_bits, gw_bits, experts, bias=None, shared=(),
                  shared_gate_bits=None, logit_bias=None):
    """Whole block: route -> experts -> combine (+ shared).  Returns
    (inds, weights, y [N,K,D] float64, out [N,D] float64)."""
    logits = router_logits(x_bits, gw_bits, logit_bias)
    inds, w = route(spec, logits, bias)
    y = switch_glu_f64(x_bits, inds, experts)
    sh = None
    if shared:
        x = bf16_to_f32(x_bits)
        sh = sum(expert_ffn_f64(x, s) for s in shared)
        if shared_gate_bits is not None:
            gl = router_logits(x_bits, shared_gate_bits)[:, 0].astype(np.float64)
            sh = sh * (1.0 / (1.0 + np.exp(-gl)))[:, None]
    return inds, w, y, combine_f64(y, w, sh)
