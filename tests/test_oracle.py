"""Pins of the CPU oracle: every oracle function is checked against something
that does not restate its own formula -- a library routine, a closed form, a
brute-force enumeration, an invariant, or a known answer from the reference's
own tests.  CPU only.
"""

import math

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import pmoe_oracle as O


def bits_of(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- bf16

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-20, 20, 100000)
    # exact ties: low 16 bits 0x8000 with even and odd upper halves
    ties = (np.arange(0x3F80, 0x3F90, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x.astype(np.float32), ties, np.float32([0.0, -0.0, 1e-40, -1e-40])])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_round(x), ref)


def test_bf16_to_f32_exact():
    b = np.arange(0, 65536, 7, dtype=np.uint16)
    f = O.bf16_to_f32(b)
    ref = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(bits_of(f), bits_of(ref))


# ---------------------------------------------------------------- exp

def test_pexp_within_2ulp_of_float64_exp():
    x = np.linspace(-85.9, 88.0, 400001).astype(np.float32)
    got = O.pexp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) <= 2 * ulp).all()


def test_pexp_special_values():
    assert O.pexp(np.float32(0.0)) == 1.0
    assert abs(float(O.pexp(np.float32(math.log(2.0)))) - 2.0) <= 2.0 ** -22
    assert O.pexp(np.float32(-100.0)) == 0.0
    assert np.isinf(O.pexp(np.float32(100.0)))
    # the C restatement is bit-identical
    for v in np.linspace(-86, 88, 997).astype(np.float32):
        assert np.float32(C.lib().pmo_pexp(float(v))) == O.pexp(v)


# ---------------------------------------------------------------- router

def test_router_logits_float64_bound():
    rng = np.random.default_rng(1)
    xb = O.bf16_round(rng.standard_normal((6, 4096), dtype=np.float32))
    wb = O.bf16_round(rng.standard_normal((40, 4096), dtype=np.float32) * np.float32(0.02))
    got = O.router_logits(xb, wb).astype(np.float64)
    x = O.bf16_to_f32(xb).astype(np.float64)
    w = O.bf16_to_f32(wb).astype(np.float64)
    ref = x @ w.T
    mag = np.abs(x) @ np.abs(w).T
    # fp32 summation of 4096 exact products: error <= (terms per lane + 6) ulps of the magnitude
    assert (np.abs(got - ref) <= (64 + 6) * 2.0 ** -24 * mag).all()


def test_router_logits_integer_inputs_exact():
    # small integers: every partial sum is exact, so any order gives x @ w.T
    rng = np.random.default_rng(2)
    x = rng.integers(-8, 9, (5, 1024)).astype(np.float32)
    w = rng.integers(-8, 9, (17, 1024)).astype(np.float32)
    got = O.router_logits(O.bf16_round(x), O.bf16_round(w))
    assert np.array_equal(got, (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32))


def test_router_logits_single_term_and_bias():
    xb = O.bf16_round(np.zeros((2, 1536), np.float32))
    xb[0, 777] = O.bf16_round(np.float32([1.5]))[0]
    xb[1, 3] = O.bf16_round(np.float32([-2.0]))[0]
    wb = O.bf16_round(np.arange(3 * 1536, dtype=np.float32).reshape(3, 1536) / np.float32(4096))
    bias = np.float32([0.25, -1.0, 3.0])
    got = O.router_logits(xb, wb, bias)
    w = O.bf16_to_f32(wb)
    assert np.array_equal(got[0], np.float32(1.5) * w[:, 777] + bias)
    assert np.array_equal(got[1], np.float32(-2.0) * w[:, 3] + bias)


def test_router_logits_c_restatement_bit_exact():
    rng = np.random.default_rng(3)
    for n, d, e in [(3, 1024, 32), (2, 7168, 384), (4, 1000, 9)]:
        xb = O.bf16_round(rng.standard_normal((n, d), dtype=np.float32))
        wb = O.bf16_round(rng.standard_normal((e, d), dtype=np.float32) * np.float32(0.02))
        assert np.array_equal(O.router_logits(xb, wb), C.router_logits(xb, wb))


# ---------------------------------------------------------------- softmax top-k

def brute_topk(row, k):
    return [i for _, i in sorted(((-float(v), i) for i, v in enumerate(row)))[:k]]


@pytest.mark.parametrize("e,k", [(8, 2), (32, 4), (128, 8), (7, 7), (512, 10)])
def test_softmax_topk_brute_force(e, k):
    rng = np.random.default_rng(e * k)
    logits = rng.standard_normal((20, e), dtype=np.float32)
    logits[0, : min(e, 5)] = logits[0, min(e, 5) - 1]     # ties -> lower id first
    logits[1] = np.round(logits[1])                        # many ties
    inds, w = O.softmax_topk(logits, k, True)
    for r in range(logits.shape[0]):
        assert inds[r].tolist() == brute_topk(logits[r], k)
    # weights: float64 softmax over the picks, sum to 1
    sel = np.take_along_axis(logits.astype(np.float64), inds.astype(np.int64), axis=1)
    ref = np.exp(sel - sel.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.allclose(w, ref, rtol=2e-6, atol=1e-7)
    assert np.allclose(w.sum(1), 1.0, atol=2e-6)


def test_softmax_topk_without_renorm_is_full_softmax_entries():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((8, 64), dtype=np.float32)
    inds, w = O.softmax_topk(logits, 6, False)
    p = torch.softmax(torch.from_numpy(logits).double(), -1).numpy()
    assert np.allclose(w, np.take_along_axis(p, inds.astype(np.int64), 1), rtol=2e-6, atol=1e-8)


def test_topk_of_logits_equals_topk_of_softmax():
    # streaming.py:2068-2073: the router's top-k can be taken on logits
    rng = np.random.default_rng(10)
    logits = rng.standard_normal((50, 128), dtype=np.float32)
    inds, _ = O.softmax_topk(logits, 8)
    p = torch.softmax(torch.from_numpy(logits).double(), -1)
    ref = torch.topk(p, 8, dim=-1).indices.numpy()
    assert np.array_equal(np.sort(inds, 1), np.sort(ref, 1))


def test_reference_block_restated_with_torch():
    # tests/test_stream.py:191-196 (softmax(precise) -> top-k -> take ->
    # renorm), written in torch float64: same index sets, weights to 2e-6.
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((40, 32), dtype=np.float32)
    gates = torch.softmax(torch.from_numpy(logits).double(), -1)
    idx = torch.topk(gates, 4, -1).indices
    scores = torch.take_along_dim(gates, idx, -1)
    scores = scores / scores.sum(-1, keepdim=True)
    inds, w = O.softmax_topk(logits, 4, True)
    assert np.array_equal(inds, idx.numpy())
    assert np.allclose(w, scores.numpy(), rtol=2e-6, atol=1e-8)


def test_softmax_topk_c_restatement_bit_exact():
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((9, 384), dtype=np.float32)
    for norm in (True, False):
        a = O.softmax_topk(logits, 8, norm)
        b = C.softmax_topk(logits, 8, norm)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# ---------------------------------------------------------------- sigmoid grouped top-k

def brute_group_topk(l, bias, n_group, topk_group, k, norm, scale):
    """DeepSeek-V3 noaux_tc written out per expert with Python sorting."""
    e = len(l)
    gs = e // n_group
    sig = [1.0 / (1.0 + math.exp(-float(v))) for v in l]
    c = [s + float(b) for s, b in zip(sig, bias)]
    if n_group > 1:
        gscore = [sum(sorted(c[g * gs:(g + 1) * gs], reverse=True)[:2]) for g in range(n_group)]
        keep = [g for _, g in sorted((-s, g) for g, s in enumerate(gscore))[:topk_group]]
        c = [c[i] if i // gs in keep else 0.0 for i in range(e)]
    picks = [i for _, i in sorted((-v, i) for i, v in enumerate(c))[:k]]
    w = [sig[i] for i in picks]
    if norm:
        s = sum(w)
        w = [x / s for x in w]
    return picks, [x * scale for x in w]


@pytest.mark.parametrize("e,ng,tg,k", [(16, 4, 2, 3), (64, 8, 4, 8), (384, 8, 4, 8), (24, 1, 1, 5)])
def test_sigmoid_group_topk_brute_force(e, ng, tg, k):
    rng = np.random.default_rng(e + ng)
    logits = rng.standard_normal((12, e), dtype=np.float32)
    bias = (rng.standard_normal(e, dtype=np.float32) * np.float32(0.3)).astype(np.float32)
    inds, w = O.sigmoid_group_topk(logits, bias, ng, tg, k, True, 2.5)
    for r in range(logits.shape[0]):
        picks, ref_w = brute_group_topk(logits[r], bias, ng, tg, k, True, 2.5)
        assert inds[r].tolist() == picks
        assert np.allclose(w[r], ref_w, rtol=2e-6)
    assert np.allclose(w.sum(1), 2.5, rtol=2e-6)


def test_sigmoid_single_group_is_plain_topk():
    rng = np.random.default_rng(13)
    logits = rng.standard_normal((10, 96), dtype=np.float32)
    bias = np.zeros(96, np.float32)
    inds, _ = O.sigmoid_group_topk(logits, bias, 1, 1, 6, True, 1.0)
    ref, _ = O.softmax_topk(logits, 6)
    assert np.array_equal(inds, ref)           # sigmoid is monotone in the logit


def test_sigmoid_c_restatement_bit_exact():
    rng = np.random.default_rng(14)
    logits = rng.standard_normal((7, 384), dtype=np.float32)
    bias = (rng.standard_normal(384, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    a = O.sigmoid_group_topk(logits, bias, 8, 4, 8, True, 2.5)
    b = C.sigmoid_group_topk(logits, bias, 8, 4, 8, True, 2.5)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_unit_mass_known_answer():
    # tests/test_moe_gate_routing.py:28-34
    scaled = np.array([[0.5 * 2.5, 0.3 * 2.5, 0.2 * 2.5]], dtype=np.float32)
    u = O.unit_mass(scaled)
    assert np.allclose(u.sum(axis=-1), 1.0)
    assert np.allclose(u, [[0.5, 0.3, 0.2]])


# ---------------------------------------------------------------- dispatch

def brute_dispatch(ids, e):
    flat = [int(v) for v in np.asarray(ids).reshape(-1)]
    order = [r for ex in range(e) for r, v in enumerate(flat) if v == ex]
    counts = [flat.count(ex) for ex in range(e)]
    return order, counts


@pytest.mark.parametrize("rows,e", [(0, 4), (1, 4), (64, 8), (500, 16), (2048, 128)])
def test_dispatch_brute_force_and_invariants(rows, e):
    rng = np.random.default_rng(rows + e)
    ids = rng.integers(0, e, rows).astype(np.int32)
    d = O.dispatch(ids, e)
    order, counts = brute_dispatch(ids, e)
    assert d.order.tolist() == order
    assert d.counts.tolist() == counts
    assert d.offsets[0] == 0 and d.offsets[-1] == rows
    assert sorted(d.order.tolist()) == list(range(rows))          # a permutation
    assert (np.diff(ids[d.order]) >= 0).all() if rows else True   # grouped by expert
    assert (d.inv[d.order] == np.arange(rows)).all()
    assert d.active.tolist() == [x for x in range(e) if counts[x]]


# ---------------------------------------------------------------- quant format

def pack6_bytes(vals):
    """mlx's 6-bit layout written byte-wise: 4 values in 3 bytes."""
    out = []
    for i in range(0, len(vals), 4):
        q0, q1, q2, q3 = (int(v) for v in vals[i:i + 4])
        out += [q0 | ((q1 & 3) << 6), (q1 >> 2) | ((q2 & 15) << 4), (q2 >> 4) | (q3 << 2)]
    return np.frombuffer(bytes(out), dtype="<u4")


def test_pack4_known_answer():
    q = np.arange(8, dtype=np.uint8)[None, :]
    assert O.pack_rows(q, 4)[0, 0] == 0x76543210


def test_pack6_matches_bytewise_layout():
    rng = np.random.default_rng(15)
    q = rng.integers(0, 64, (5, 128)).astype(np.uint8)
    w = O.pack_rows(q, 6)
    for r in range(5):
        assert np.array_equal(w[r], pack6_bytes(q[r]))
    v = [int(t) for t in q[0, :6]]
    assert w[0, 0] == (v[0] | v[1] << 6 | v[2] << 12 | v[3] << 18 | v[4] << 24 | (v[5] & 0x3) << 30)


@pytest.mark.parametrize("bits", [4, 6])
def test_pack_unpack_round_trip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, (9, 256)).astype(np.uint8)
    assert np.array_equal(O.unpack_rows(O.pack_rows(q, bits), bits, 256), q)


@pytest.mark.parametrize("bits", [4, 6])
def test_quantize_error_bound(bits):
    rng = np.random.default_rng(20 + bits)
    w = rng.standard_normal((32, 512), dtype=np.float32) * np.float32(0.02)
    qt = O.quantize(w, bits)
    deq = O.dequant_f64(qt)
    s = np.repeat(O.bf16_to_f32(qt.scales).astype(np.float64), 64, axis=1)
    g = w.reshape(32, 8, 64)
    span = np.repeat((np.abs(g).max(-1)).astype(np.float64), 64, axis=1)
    # half a step, plus what bf16 rounding of scale and bias can move a level
    bound = 0.5 * s + 2.0 ** -8 * span * (1 + (1 << bits))
    assert (np.abs(deq - w) <= bound).all()


def unpack_bytewise(words, bits):
    """Unpack rows of little-endian u32 words byte by byte (mlx layouts:
    two nibbles per byte, low first; or 4 six-bit values per 3 bytes)."""
    out = []
    for row in words:
        by = np.asarray(row, "<u4").tobytes()
        vals = []
        if bits == 4:
            for b0 in by:
                vals += [b0 & 15, b0 >> 4]
        else:
            for i in range(0, len(by), 3):
                b0, b1, b2 = by[i], by[i + 1], by[i + 2]
                vals += [b0 & 63, (b0 >> 6) | ((b1 & 15) << 2), (b1 >> 4) | ((b2 & 3) << 4), b2 >> 2]
        out.append(vals)
    return np.array(out, np.float32)


@pytest.mark.parametrize("bits", [4, 6])
def test_dequant_matches_torch_closed_form(bits):
    rng = np.random.default_rng(30 + bits)
    w = rng.standard_normal((16, 256), dtype=np.float32) * np.float32(0.05)
    qt = O.quantize(w, bits)
    q = unpack_bytewise(qt.weight, bits)
    assert np.array_equal(q, O.unpack_rows(qt.weight, bits, 256).astype(np.float32))
    s = torch.from_numpy(qt.scales.view(np.int16)).view(torch.bfloat16).float().repeat_interleave(64, 1)
    b = torch.from_numpy(qt.biases.view(np.int16)).view(torch.bfloat16).float().repeat_interleave(64, 1)
    ref = (s * torch.from_numpy(q) + b).to(torch.bfloat16)
    assert np.array_equal(O.dequant_bf16(qt), ref.view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------- expert FFN + combine

def test_expert_ffn_matches_torch_float64():
    spec = O.LayerSpec(256, 4, 128, 2)
    rng = np.random.default_rng(40)
    ex = O.make_expert(rng, 256, 128, 4)
    x = O.bf16_to_f32(O.bf16_round(rng.standard_normal((5, 256), dtype=np.float32)))
    got = O.expert_ffn_f64(x, ex)
    wg = torch.from_numpy(O.dequant_f64(ex.gate))
    wu = torch.from_numpy(O.dequant_f64(ex.up))
    wd = torch.from_numpy(O.dequant_f64(ex.down))
    xt = torch.from_numpy(x.astype(np.float64))
    ref = torch.nn.functional.linear(torch.nn.functional.silu(xt @ wg.T) * (xt @ wu.T), wd)
    assert np.allclose(got, ref.numpy(), rtol=1e-12, atol=1e-15)
    del spec


def test_switch_glu_rows_in_token_slot_order():
    spec = O.LayerSpec(256, 6, 128, 3)
    gw, experts, _, _, _ = O.make_layer(spec, seed=3)
    rng = np.random.default_rng(41)
    xb = O.bf16_round(rng.standard_normal((4, 256), dtype=np.float32))
    inds = np.array([[5, 0, 2], [2, 2, 1], [0, 4, 3], [1, 5, 0]], np.int32)
    y = O.switch_glu_f64(xb, inds, experts)
    x = O.bf16_to_f32(xb)
    for n in range(4):
        for k in range(3):
            assert np.allclose(y[n, k], O.expert_ffn_f64(x[n:n + 1], experts[int(inds[n, k])])[0])


def test_combine_closed_form():
    rng = np.random.default_rng(42)
    y = rng.standard_normal((3, 4, 16))
    w = rng.random((3, 4))
    sh = rng.standard_normal((3, 16))
    got = O.combine_f64(y, w, sh)
    for n in range(3):
        ref = sh[n] + sum(w[n, k] * y[n, k] for k in range(4))
        assert np.allclose(got[n], ref)


def test_combine_f32_fixed_order_known_answers():
    """The fp32 combine accumulates in k order, then the shared term:
    1 + 2^-25 rounds back to 1 in float32, so [1, 2^-25, -1] sums to 0 in
    that order (2^-25 in any order that adds the small term last)."""
    y = np.zeros((2, 3, 64), np.float32)
    y[0, :, 0] = [1.0, 2.0 ** -25, -1.0]
    y[1, :, 0] = [2.0 ** -25, 1.0, -1.0]
    w = np.ones((2, 3), np.float32)
    got = O.bf16_to_f32(O.combine_f32(y, w))
    assert got[0, 0] == 0.0 and got[1, 0] == 0.0
    sh = np.zeros((2, 64), np.float32)
    sh[:, 0] = 2.0 ** -25
    got = O.bf16_to_f32(O.combine_f32(y, w, sh))
    assert got[0, 0] == np.float32(2.0 ** -25)      # shared added after the routed sum
    # exact power-of-two weights reproduce the closed form bit for bit
    rng = np.random.default_rng(5)
    yb = O.bf16_to_f32(O.bf16_round(rng.standard_normal((4, 2, 128), dtype=np.float32)))
    w2 = np.array([[0.5, 0.25]] * 4, np.float32)
    ref = O.bf16_round((yb[:, 0] * 0.5 + yb[:, 1] * 0.25).astype(np.float32))
    assert np.array_equal(O.combine_f32(yb, w2), ref)
    # and sigmoid-gated shared terms agree with the float64 closed form
    yf = rng.standard_normal((3, 5, 256)).astype(np.float32)
    wf = rng.random((3, 5), dtype=np.float32)
    shf = rng.standard_normal((3, 256)).astype(np.float32)
    sw = O.psigmoid(rng.standard_normal(3, dtype=np.float32))
    got = O.bf16_to_f32(O.combine_f32(yf, wf, shf, sw))
    ref = O.combine_f64(yf, wf, shf.astype(np.float64) * sw[:, None])
    assert np.abs(got - ref).max() <= 2.0 ** -8 * np.abs(ref).max()


@pytest.mark.parametrize("bits", [4, 6])
def test_c_expert_ffn_matches_oracle(bits):
    spec = O.LayerSpec(1024, 2, 512, 1, bits=bits)
    _, experts, _, _, _ = O.make_layer(spec, seed=4)
    x = O.bf16_to_f32(O.bf16_round(np.random.default_rng(44).standard_normal((1, 1024),
                                                                           dtype=np.float32)))
    got = C.expert_ffn(experts[1], x[0], 1024, 512, bits)
    ref = O.expert_ffn_f64(x, experts[1])[0]
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_c_decode_layer_matches_oracle():
    spec = O.LayerSpec(1024, 16, 256, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=2)
    xb = O.bf16_round(np.random.default_rng(43).standard_normal((3, 1024), dtype=np.float32))
    layer = C.DecodeLayer(gw, [experts[e] for e in range(16)], 1024, 256, 4, 4)
    inds, w, out = layer(xb)
    ri, rw, _, ref = O.moe_layer_f64(spec, xb, gw, experts)
    assert np.array_equal(inds, ri) and np.array_equal(w, rw)
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


# ---------------------------------------------------------------- slot policy

def test_stitch_set_is_unevictable():
    # test_stitch.py:53-58: a full stitch set is not evictable
    pol = O.SlotPolicy(64)
    assert pol.stitch([0, 1], 32)
    assert pol.table(1, 32).tolist() == list(range(32, 64))   # slot = layer*E + e
    before = set(pol.stitch_keys)
    assert pol._alloc(True) is None
    assert set(pol.stitch_keys) == before and len(pol.lru) == 64


def test_admit_installs_refreshes_and_counts_hits():
    # test_flow.py:88-118: misses install and fill the table; a resident id
    # counts as a hit and becomes most recent
    pol = O.SlotPolicy(40)
    pol.step(0, [7, 3])
    t = pol.table(0, 16)
    assert t[3] >= 0 and t[7] >= 0 and pol.misses == 2
    pol.step(0, [0])
    assert list(pol.lru)[-1] == (0, 0)
    hits = pol.hits
    pol.step(0, [3])
    assert pol.hits == hits + 1 and list(pol.lru)[-1] == (0, 3)


def test_every_slot_accounted_once():
    # test_prefill_slab.py:79-99
    pol = O.SlotPolicy(48)
    rng = np.random.default_rng(44)
    for _ in range(200):
        pol.step(int(rng.integers(0, 3)), rng.choice(100, 8, replace=False))
        used = list(pol.slot_of.values())
        assert len(used) == len(set(used))
        assert set(used).isdisjoint(pol.free)
        assert sorted(used + pol.free) == list(range(48))
        assert len(pol.lru) <= pol.budget


def test_plain_lru_brute_force():
    """With LFRU off the policy is plain LRU over budget entries; compare with
    a list-based LRU written independently."""
    slots = 40
    pol = O.SlotPolicy(slots, lfru=False)
    budget = slots - max(4, int(slots * 0.1))
    lru: list = []
    rng = np.random.default_rng(45)
    for _ in range(300):
        ids = sorted(set(rng.integers(0, 80, 6).tolist()))
        pol.step(0, ids)
        hits = [e for e in ids if e in lru]
        for e in hits:
            lru.remove(e)
            lru.append(e)
        for e in ids:
            if e not in hits:
                lru.append(e)
                while len(lru) > budget:
                    victim = next(v for v in lru if v not in ids)
                    lru.remove(victim)
        assert [e for (_, e) in pol.lru] == lru


class _OracleSlots:
    """slot_kats adapter over the oracle's SlotPolicy (layer 0)."""

    def __init__(self, slots, lfru=True, stage=None):
        self.pol = O.SlotPolicy(slots, lfru=lfru)
        if stage is not None:
            self.pol.set_stage(*stage)

    def step(self, ids):
        return self.pol.step(0, ids)[1]

    def prefill(self, ids):
        return self.pol.step_prefill(0, ids)

    def compute_row(self, ticket):
        row = self.pol.compute_row(ticket, 64)
        return {e: int(s) for e, s in enumerate(row) if s >= 0}

    def done(self, ticket):
        self.pol.prefill_done(ticket)

    def table(self):
        return {e: int(s) for e, s in enumerate(self.pol.table(0, 64)) if s >= 0}

    @property
    def evictions(self):
        return self.pol.evictions

    @property
    def hits(self):
        return self.pol.hits

    @property
    def misses(self):
        return self.pol.misses

    def admit(self, ids):
        return self.pol.admit(0, ids)

    def install(self, ids):
        self.pol.install(0, ids)


def test_speculation_known_answer():
    """Guesses take free slots only, a fetch claims them as hits with no
    read, and hands back its layer's unclaimed guesses (cache.py:2853,
    :2379-2386)."""
    from tests import slot_kats
    kat = slot_kats.SPECULATION
    pol = O.SlotPolicy(kat["slots"])
    pol.step(0, kat["warm"])
    assert pol.speculate(0, kat["guesses"], kat["max_staged"]) == kat["started"]
    before = set(e for (_, e) in pol.lru)
    _, placed = pol.step(0, kat["fetch"])
    assert placed == kat["fetch_placed"]
    assert sorted(before - set(e for (_, e) in pol.lru)) == kat["evicted"]
    assert (pol.hits, pol.misses, pol.evictions) == (kat["hits"], kat["misses"], 3)
    pol.settle()
    assert pol.free == kat["free_after_settle"]


def test_flow_admit_known_answer():
    from tests import slot_kats
    slot_kats.run_flow_kat(_OracleSlots(8), slot_kats.FLOW_ADMIT)


@pytest.mark.parametrize("name", ["LFRU_SECOND_CHANCE", "PINNED_OVER_BUDGET"])
def test_lfru_known_answer(name):
    """Hand-worked traces of the LFRU second chance (cache.py:2236-2291)."""
    from tests import slot_kats
    kat = getattr(slot_kats, name)
    slot_kats.run_decode_kat(_OracleSlots(kat["slots"]), kat)


def test_plain_lru_known_answer():
    from tests import slot_kats
    kat = slot_kats.PLAIN_LRU
    slot_kats.run_decode_kat(_OracleSlots(kat["slots"], lfru=False), kat)


@pytest.mark.parametrize("name", ["PREFILL_AFTER_DECODE", "PREFILL_COLD"])
def test_prefill_known_answer(name):
    """Prefill groups never evict and leave the decode hot set's recency
    alone (cache.py:2347-2453 with prefill=True, _install soft :2306-2312)."""
    from tests import slot_kats
    kat = getattr(slot_kats, name)
    slot_kats.run_prefill_kat(_OracleSlots(kat["slots"], stage=kat["stage"]), kat)


class _ListLFRU:
    """An LFRU slab written as a plain list (LRU first) plus a counter dict,
    from the reference's description alone (cache.py:2236-2291 second chance,
    :2367-2378 reuse credit, :1118-1159 slot choice, :991 free list)."""

    def __init__(self, slots, scan=8, cap=8):
        self.free = list(range(slots))[::-1]
        self.budget = slots - max(4, int(slots * 0.1))
        self.scan, self.cap = scan, cap
        self.order, self.count, self.where = [], {}, {}
        self.evicted = 0
        self.reprieves = 0

    def _drop(self, e):
        self.order.remove(e)
        del self.count[e]
        self.evicted += 1
        return self.where.pop(e)

    def step(self, ids):
        ids = sorted(set(int(i) for i in ids))
        keep = set()
        fresh = []
        for e in ids:
            if e in self.where:
                self.order.remove(e)
                self.order.append(e)
                self.count[e] = min(self.cap, self.count[e] + 1)
                keep.add(self.where[e])
            else:
                fresh.append(e)
        got = []
        for e in fresh:
            if self.free:
                slot = self.free.pop()
            else:
                cand = [v for v in self.order if self.where[v] not in keep]
                if not cand:
                    continue
                slot = self._drop(cand[0])
            keep.add(slot)
            got.append((e, slot))
        for e, slot in got:
            self.where[e] = slot
            self.count[e] = 0
            self.order.append(e)
            while len(self.order) > max(self.budget, 1):
                for _ in range(self.scan):
                    if len(self.order) <= 1 or self.count[self.order[0]] == 0:
                        break
                    head = self.order.pop(0)
                    self.count[head] //= 2
                    self.order.append(head)
                    self.reprieves += 1
                cand = [v for v in self.order if self.where[v] not in keep]
                if not cand:
                    break
                self.free.append(self._drop(cand[0]))
        return got


@pytest.mark.parametrize("seed,slots,experts,k", [(0, 24, 60, 4), (1, 40, 100, 8), (2, 12, 30, 3)])
def test_lfru_matches_list_implementation(seed, slots, experts, k):
    """The oracle's LFRU against the list-plus-counter restatement over
    random Zipf-skewed traces (so reuse credit and second chances occur)."""
    rng = np.random.default_rng(seed)
    pop = 1.0 / np.arange(1, experts + 1) ** 1.1
    pop /= pop.sum()
    pol = O.SlotPolicy(slots)
    ref = _ListLFRU(slots)
    for _ in range(600):
        ids = rng.choice(experts, k, replace=False, p=pop).tolist()
        _, placed = pol.step(0, ids)
        got = ref.step(ids)
        assert placed == got
        assert [e for (_, e) in pol.lru] == ref.order
        assert {e: pol.freq.get((0, e), 0) for (_, e) in pol.lru} == ref.count
    assert pol.evictions == ref.evicted
    assert ref.reprieves > 50      # the second-chance branch is exercised


def test_prefill_ahead_known_answer():
    """Prefill-time prediction (cache.py:2580-2650): free slots above a
    floor, then stage slots above a floor, never an eviction; the next
    layer's prefill group claims what it routes and the rest is handed back
    (hand-worked trace in tests/slot_kats.py)."""
    from tests import slot_kats
    kat = slot_kats.PREFILL_AHEAD
    pol = O.SlotPolicy(kat["slots"])
    pol.set_stage(*kat["stage"])
    pol.step(0, kat["warm"])
    assert pol.prefill_ahead(1, kat["ahead"], kat["free_floor"], kat["stage_floor"]) == \
        kat["started"]
    ticket, placed, unplaced = pol.step_prefill(1, kat["prefill"])
    assert placed == kat["prefill_placed"] and unplaced == 0
    row = pol.compute_row(ticket, 64)
    assert {e: int(s) for e, s in enumerate(row) if s >= 0 and e in kat["prefill"]} == \
        kat["compute_row"]
    pol.settle()
    pol.prefill_done(ticket)
    assert {e: int(s) for e, s in enumerate(pol.table(1, 64)) if s >= 0} == kat["after"]
    assert (pol.hits, pol.misses, pol.evictions) == (kat["hits"], kat["misses"],
                                                     kat["evictions"])
    assert pol.free == kat["free_after"] and pol.stage_free == kat["stage_after"]


def test_prefill_ahead_floors_and_skips():
    """Resident, staged and repeated ids are skipped; nothing is started
    when both lists are at their floors."""
    pol = O.SlotPolicy(16)
    pol.set_stage(16, 4)
    pol.step(0, list(range(12)))                  # free [15, 14, 13, 12]
    assert pol.prefill_ahead(0, [3, 20, 20, 21], 2, 4) == [(20, 12), (21, 13)]
    assert pol.prefill_ahead(0, [20, 22], 2, 4) == []   # 20 staged; free at the floor
    assert pol.prefill_ahead(0, [22, 23], 2, 3) == [(22, 16)]
