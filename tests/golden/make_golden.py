"""Write the golden fixtures of the routed-expert path (tests/golden/*.npz).

Run from the repository root:  python tests/golden/make_golden.py

The fixtures are produced by the CPU oracle (oracle/pmoe_oracle.py) on the
seeded workloads below and committed, so later changes to the oracle (or to
numpy's generators) show up as fixture mismatches in tests/test_golden.py.
Expert weights are regenerated from their seeds rather than stored (they are
megabytes); a SHA-256 of their packed bytes is stored instead.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import pmoe_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent


def experts_digest(experts: dict) -> str:
    h = hashlib.sha256()
    for e in sorted(experts):
        ex = experts[e]
        for qt in (ex.gate, ex.up, ex.down):
            h.update(qt.weight.tobytes())
            h.update(qt.scales.tobytes())
            h.update(qt.biases.tobytes())
    return h.hexdigest()


def tiny_layer():
    """Config 1: D1024, E32, I512, top-4 softmax+renorm, 4-bit g64, 64
    tokens, seed 0."""
    spec = O.LayerSpec(1024, 32, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=0)
    xb = O.bf16_round(np.random.default_rng(0).standard_normal((64, 1024), dtype=np.float32))
    logits = O.router_logits(xb, gw)
    inds, w, y, out = O.moe_layer_f64(spec, xb, gw, experts)
    np.savez_compressed(
        OUT / "tiny_layer.npz", x_bits=xb, gate_bits=gw, logits=logits, inds=inds, weights=w,
        out=out.astype(np.float32), y=y.astype(np.float32)[:2],
        experts_sha256=np.array(experts_digest(experts)))


def routing_sigmoid():
    """DeepSeek-V3-style routing on random logits: 384 experts, 8 groups,
    top-4 groups, top-8, scale 2.5."""
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((16, 384), dtype=np.float32)
    bias = (rng.standard_normal(384, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    inds, w = O.sigmoid_group_topk(logits, bias, 8, 4, 8, True, 2.5)
    np.savez_compressed(OUT / "routing_sigmoid.npz", logits=logits, bias=bias, inds=inds,
                        weights=w)


def routing_softmax():
    """Softmax top-k with ties and without renormalisation, 512 experts, k 10."""
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((16, 512), dtype=np.float32)
    logits[0, :12] = logits[0].max() + 1.0   # 12-way tie at the top
    i1, w1 = O.softmax_topk(logits, 10, True)
    i2, w2 = O.softmax_topk(logits, 10, False)
    np.savez_compressed(OUT / "routing_softmax.npz", logits=logits, inds=i1, weights=w1,
                        inds_nonorm=i2, weights_nonorm=w2)


def quant_format():
    """4- and 6-bit affine g64 packing of a 64 x 256 matrix."""
    rng = np.random.default_rng(6)
    w = rng.standard_normal((64, 256), dtype=np.float32) * np.float32(0.02)
    w[1, :64] = 0.5
    arrs = {"w": w}
    for bits in (4, 6):
        qt = O.quantize(w, bits)
        arrs[f"q{bits}"] = qt.weight
        arrs[f"s{bits}"] = qt.scales
        arrs[f"b{bits}"] = qt.biases
        arrs[f"deq{bits}"] = O.dequant_bf16(qt)
    np.savez_compressed(OUT / "quant_format.npz", **arrs)


def dispatch():
    """Stable dispatch of 2048 tokens x top-8 over 128 experts, skewed."""
    rng = np.random.default_rng(7)
    p = np.exp(rng.standard_normal(128))
    p /= p.sum()
    ids = rng.choice(128, size=(2048, 8), p=p).astype(np.int32)
    d = O.dispatch(ids, 128)
    np.savez_compressed(OUT / "dispatch.npz", ids=ids, order=d.order, counts=d.counts,
                        offsets=d.offsets, inv=d.inv, active=d.active)


def slot_trace():
    """Config 4 slot table: 96 slots, 384 experts, Zipf(1.1) popularity over a
    fixed permutation, 8 distinct experts per step, 300 steps."""
    trace = zipf_trace(seed=0, steps=300, n_experts=384, k=8)
    pol = O.SlotPolicy(96)
    tables, stats = [], []
    for ids in trace:
        pol.step(0, ids)
        tables.append(pol.table(0, 384))
        stats.append((pol.hits, pol.misses, pol.evictions))
    np.savez_compressed(OUT / "slot_trace.npz", trace=np.array(trace, np.int32),
                        tables=np.array(tables, np.int32), stats=np.array(stats, np.int64))


def zipf_trace(seed: int, steps: int, n_experts: int, k: int):
    """k distinct expert ids per step, popularity rank r drawn ~ 1/r^1.1,
    ranks mapped through a fixed random permutation."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_experts)
    p = 1.0 / np.arange(1, n_experts + 1) ** 1.1
    p /= p.sum()
    out = []
    for _ in range(steps):
        ranks = rng.choice(n_experts, size=k, replace=False, p=p)
        out.append(sorted(int(perm[r]) for r in ranks))
    return out


if __name__ == "__main__":
    tiny_layer()
    routing_sigmoid()
    routing_softmax()
    quant_format()
    dispatch()
    slot_trace()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
