"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py).  CPU only."""

from pathlib import Path

import numpy as np

from oracle import pmoe_oracle as O
from tests.golden.make_golden import experts_digest, zipf_trace

G = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(G / name, allow_pickle=False)


def test_tiny_layer_fixture():
    f = load("tiny_layer.npz")
    spec = O.LayerSpec(1024, 32, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=0)
    assert str(f["experts_sha256"]) == experts_digest(experts), "seeded expert weights changed"
    assert np.array_equal(gw, f["gate_bits"])
    logits = O.router_logits(f["x_bits"], gw)
    assert np.array_equal(logits, f["logits"])
    inds, w, y, out = O.moe_layer_f64(spec, f["x_bits"], gw, experts)
    assert np.array_equal(inds, f["inds"]) and np.array_equal(w, f["weights"])
    assert np.array_equal(out.astype(np.float32), f["out"])
    assert np.array_equal(y.astype(np.float32)[:2], f["y"])


def test_routing_fixtures():
    f = load("routing_sigmoid.npz")
    inds, w = O.sigmoid_group_topk(f["logits"], f["bias"], 8, 4, 8, True, 2.5)
    assert np.array_equal(inds, f["inds"]) and np.array_equal(w, f["weights"])
    f = load("routing_softmax.npz")
    i1, w1 = O.softmax_topk(f["logits"], 10, True)
    i2, w2 = O.softmax_topk(f["logits"], 10, False)
    assert np.array_equal(i1, f["inds"]) and np.array_equal(w1, f["weights"])
    assert np.array_equal(i2, f["inds_nonorm"]) and np.array_equal(w2, f["weights_nonorm"])
    assert f["inds"][0].tolist()[:10] == list(range(10))   # tied logits -> lowest ids


def test_quant_fixture():
    f = load("quant_format.npz")
    for bits in (4, 6):
        qt = O.quantize(f["w"], bits)
        assert np.array_equal(qt.weight, f[f"q{bits}"])
        assert np.array_equal(qt.scales, f[f"s{bits}"])
        assert np.array_equal(qt.biases, f[f"b{bits}"])
        assert np.array_equal(O.dequant_bf16(qt), f[f"deq{bits}"])


def test_dispatch_fixture():
    f = load("dispatch.npz")
    d = O.dispatch(f["ids"], 128)
    for key in ("order", "counts", "offsets", "inv", "active"):
        assert np.array_equal(getattr(d, key), f[key]), key


def test_slot_trace_fixture():
    f = load("slot_trace.npz")
    trace = zipf_trace(seed=0, steps=300, n_experts=384, k=8)
    assert np.array_equal(np.array(trace, np.int32), f["trace"])
    pol = O.SlotPolicy(96)
    for i, ids in enumerate(trace):
        pol.step(0, ids)
        assert np.array_equal(pol.table(0, 384), f["tables"][i])
        assert (pol.hits, pol.misses, pol.evictions) == tuple(f["stats"][i])
