"""GPU: the given-ids expert-per-XCD launch behind pmoe_moe_experts.

One token with eight ids (and optionally a shared expert without a gate)
runs as one launch: block group x streams column x's expert, the shared
expert's gate/up rows and down tiles are dealt over the groups, and the
last of a tile's eight group arrivals combines it.  Each column's output is
rounded to bf16 before the combine, as the three-launch path's per-slot
outputs are, and the combine runs in column order with the shared expert
last, so the outputs must equal the three-launch path's (dispatch, gate/up,
down, combine) bit for bit -- with non-resident columns (zero rows), dropped
ids (outside [0, E): left out), repeated ids, across shapes on one
workspace and under HIP-graph replay.  The tiny shape is also checked
against the oracle's float64 FFN and combine.

A one-token decode block with 8 picks that the expert-per-XCD layer does
not route (sigmoid grouped scoring, a shared expert) runs the router launch
and then this launch on its picks, combining fp32 columns: its outputs,
picks and weights must equal the grid-wide one-launch layer's and the
three-launch decode's bit for bit.
"""

import os

import numpy as np
import pytest
import torch

from oracle import pmoe_oracle as O
from tests.util import bits_to_bf16_tensor, check_close, fill_slab_gpu, slot_to_expert

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _k():
    from pagedmoe_amd import kernels
    return kernels


class _Experts:
    """n_slots random resident experts; a table of E ids mapping the first
    ids onto the slots (the rest absent)."""

    def __init__(self, hidden, inter, bits, n_slots, n_experts, seed=0):
        from pagedmoe_amd._lib import geom
        from pagedmoe_amd.slab import SlabStore
        self.g = geom(hidden, inter, bits)
        self.slab = SlabStore(self.g, n_slots, DEV)
        fill_slab_gpu(self.slab, range(n_slots), seed=seed)
        self.n_experts = n_experts
        self.hidden = hidden
        tab = np.full(n_experts, -1, np.int32)
        rng = np.random.default_rng(seed)
        self.ids_resident = rng.permutation(n_experts)[:n_slots - 1]
        tab[self.ids_resident] = np.arange(n_slots - 1, dtype=np.int32)
        self.table_np = tab
        self.table = torch.from_numpy(tab).to(DEV)
        self.shared_slot = n_slots - 1

    def x(self, seed):
        rng = np.random.default_rng(seed)
        return bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((1, self.hidden),
                                                                    dtype=np.float32)), DEV)


def _ids(ids):
    return torch.tensor([ids], dtype=torch.int32, device=DEV)


def _weights(seed, k=8):
    rng = np.random.default_rng(seed)
    w = (rng.random((1, k)) + 0.1).astype(np.float32)
    return torch.from_numpy(w / w.sum() * np.float32(2.5)).to(DEV)


def _run(ex, x, inds, w, shared, xcd):
    from pagedmoe_amd._lib import KernelTimer
    old = os.environ.get("PMOE_EXPERTS_XCD")
    os.environ["PMOE_EXPERTS_XCD"] = "1" if xcd else "0"
    try:
        with KernelTimer() as kt:
            out = _k().moe_experts(ex.g, ex.slab.buf, ex.table, ex.n_experts, x, inds, w,
                                   shared_slot=ex.shared_slot if shared else -1)
            torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["PMOE_EXPERTS_XCD"]
        else:
            os.environ["PMOE_EXPERTS_XCD"] = old
    assert ("experts_xcd" in kt.result) == xcd, kt.result
    return out.clone()


def _same(a, b, what):
    diff = (a.view(torch.int16) != b.view(torch.int16)).sum().item()
    assert diff == 0, f"{what}: {diff} outputs differ from the three-launch path"


# (hidden, inter, bits): DeepSeek-V3-shaped (4-bit 7168/2048), Qwen3-235B-
# shaped (4096/1536), the tiny C1 shape (1024/512), a 6-bit 2048/512 shape
SHAPES = [(7168, 2048, 4), (4096, 1536, 4), (1024, 512, 4), (2048, 512, 6)]


@pytest.mark.parametrize("hidden,inter,bits", SHAPES)
@pytest.mark.parametrize("shared", [True, False])
def test_experts_xcd_matches_three_launch(hidden, inter, bits, shared):
    E = 384
    ex = _Experts(hidden, inter, bits, n_slots=11, n_experts=E, seed=hidden + inter + bits)
    res = [int(i) for i in ex.ids_resident]
    absent = [i for i in range(E) if ex.table_np[i] < 0]
    cases = {
        "eight resident": res[:8],
        "absent column": res[:5] + [absent[0]] + res[5:7],
        "dropped ids": [res[0], -1, res[1], E, res[2], res[3], E + 7, res[4]],
        "repeated ids": [res[0], res[0], res[1], res[2], res[1], res[3], res[4], res[0]],
    }
    print(f"[experts_xcd] {hidden}x{inter} {bits}-bit shared={shared}", flush=True)
    for j, (name, ids) in enumerate(cases.items()):
        x = ex.x(seed=100 + j)
        inds = _ids(ids)
        w = _weights(200 + j)
        ref = _run(ex, x, inds, w, shared, xcd=False)
        got = _run(ex, x, inds, w, shared, xcd=True)
        assert torch.isfinite(got.float()).all(), name
        _same(got, ref, f"{hidden}x{inter} {bits}-bit shared={shared} {name}")
    assert _k().workspace_error(_k().moe_workspace(ex.g, 1, 8, int(shared), E, DEV)) == 0


def test_experts_xcd_vs_oracle():
    """Tiny shape with a shared expert against the oracle: float64 FFNs of
    the slab's own experts, combined with the given weights (+ shared)."""
    E = 64
    ex = _Experts(1024, 512, 4, n_slots=10, n_experts=E, seed=5)
    ids = [int(i) for i in ex.ids_resident[:8]]
    x = ex.x(seed=7)
    w = _weights(8)
    got = _run(ex, x, _ids(ids), w, True, xcd=True)
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    xf = O.bf16_to_f32(xb)
    ys = np.stack([O.expert_ffn_f64(xf, slot_to_expert(ex.slab, int(ex.table_np[i])))[0]
                   for i in ids])
    shared_y = O.expert_ffn_f64(xf, slot_to_expert(ex.slab, ex.shared_slot))
    ref = O.combine_f64(ys[None], w.cpu().numpy(), shared_y)
    check_close(got.float().cpu().numpy(), ref, "experts_xcd vs oracle")


def test_experts_xcd_across_shapes_and_graph_replay():
    """Calls of two shapes interleaved on the cached workspaces, then a
    captured sequence replayed three times with eager calls in between:
    every output equals its eager three-launch value."""
    K = _k()
    a = _Experts(7168, 2048, 4, n_slots=10, n_experts=384, seed=1)
    b = _Experts(4096, 1536, 4, n_slots=9, n_experts=128, seed=2)
    calls = []
    for j in range(6):
        ex = a if j % 2 == 0 else b
        ids = [int(i) for i in ex.ids_resident[:8]][::-1 if j % 3 else 1]
        calls.append((ex, ex.x(300 + j), _ids(ids), _weights(400 + j), j % 2 == 0))
    refs = [_run(ex, x, i, w, sh, xcd=False) for ex, x, i, w, sh in calls]
    for r in range(2):
        for (ex, x, i, w, sh), ref in zip(calls, refs):
            _same(_run(ex, x, i, w, sh, xcd=True), ref, f"eager pass {r}")
    os.environ["PMOE_EXPERTS_XCD"] = "1"
    try:
        outs = [None] * len(calls)

        def seq():
            for n, (ex, x, i, w, sh) in enumerate(calls):
                outs[n] = K.moe_experts(ex.g, ex.slab.buf, ex.table, ex.n_experts, x, i, w,
                                        shared_slot=ex.shared_slot if sh else -1)

        seq()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            seq()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            seq()
        for r in range(3):
            graph.replay()
            torch.cuda.synchronize()
            for n, ref in enumerate(refs):
                _same(outs[n], ref, f"graph replay {r}, call {n}")
            ex, x, i, w, sh = calls[r]
            _same(_run(ex, x, i, w, sh, xcd=True), refs[r], f"eager call after replay {r}")
    finally:
        del os.environ["PMOE_EXPERTS_XCD"]
    for ex in (a, b):
        for sh in (0, 1):
            assert K.workspace_error(K.moe_workspace(ex.g, 1, 8, sh, ex.n_experts, DEV)) == 0


def test_experts_xcd_split_group_is_reported_at_once():
    """Placement check of the given-ids launch, forced from the host (block
    0 reports another XCD; every block exits normally): error bit 1 is set,
    some output is NaN, the launch does not wait out the spin limit, and the
    next call is bit-exact again."""
    import time

    from pagedmoe_amd._lib import PmoeError
    K = _k()
    ex = _Experts(4096, 1536, 4, n_slots=10, n_experts=128, seed=3)
    ids = _ids([int(i) for i in ex.ids_resident[:8]])
    x, w = ex.x(11), _weights(12)
    good = _run(ex, x, ids, w, True, xcd=True)
    ws = K.moe_workspace(ex.g, 1, 8, 1, 128, DEV)
    assert K.workspace_error(ws) == 0
    print("[experts_xcd] split probe on", flush=True)
    K.set_split_probe(True)
    try:
        t0 = time.perf_counter()
        bad = _run(ex, x, ids, w, True, xcd=True)
        dt = time.perf_counter() - t0
    finally:
        K.set_split_probe(False)
    assert K.workspace_error(ws) & 2
    assert torch.isnan(bad.float()).any(), "a split group wrote only finite outputs"
    assert dt < 0.2, f"the split launch took {dt:.3f} s: a poll waited out its limit"
    with pytest.raises(PmoeError, match="different XCDs"):
        K.check_workspace_errors()
    again = _run(ex, x, ids, w, True, xcd=True)
    assert K.workspace_error(ws) == 0
    _same(again, good, "after the split probe")


def test_decode_block_routes_then_takes_the_given_ids_launch():
    """DeepSeek-V3-shaped block at batch 1 (384 experts, sigmoid + bias, 8
    groups / top-4 / top-8, scale 2.5, a shared expert): moe_block launches
    the router (routing in its last block) and the given-ids launch; equal
    to the grid-wide one-launch layer and the three-launch decode."""
    from pagedmoe_amd._lib import KernelTimer, geom
    from pagedmoe_amd.slab import SlabStore
    K = _k()
    D, E, I = 7168, 384, 2048
    g = geom(D, I, 4)
    n_res = 12
    slab = SlabStore(g, n_res + 1, DEV)
    fill_slab_gpu(slab, range(n_res + 1), seed=31)
    rng = np.random.default_rng(31)
    gate = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((E, D), dtype=np.float32)
                                            * np.float32(0.02)), DEV)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(DEV)
    table = torch.from_numpy((np.arange(E) % n_res).astype(np.int32)).to(DEV)
    rc = K.route_cfg("sigmoid", E, 8, True, 8, 4, 2.5)

    def run(fused, xcd, x):
        saved = {v: os.environ.get(v) for v in ("PMOE_DECODE_FUSED", "PMOE_EXPERTS_XCD")}
        os.environ["PMOE_DECODE_FUSED"] = fused
        os.environ["PMOE_EXPERTS_XCD"] = xcd
        try:
            with KernelTimer() as kt:
                out, inds, w = K.moe_block(g, rc, slab.buf, table, gate, x, score_bias=bias,
                                           shared_slot=n_res)
                torch.cuda.synchronize()
        finally:
            for v, old in saved.items():
                if old is None:
                    del os.environ[v]
                else:
                    os.environ[v] = old
        return out.clone(), inds.clone(), w.clone(), kt.result

    for j in range(3):
        x = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((1, D), dtype=np.float32)), DEV)
        print(f"[experts_xcd] decode block, token {j}", flush=True)
        a = run("1", "1", x)
        assert "experts_xcd" in a[3] and "router_logits" in a[3], a[3]
        b = run("1", "0", x)
        assert "decode_fused" in b[3], b[3]
        c = run("0", "1", x)
        for other, name in ((b, "grid-wide one-launch"), (c, "three-launch")):
            assert torch.equal(a[1], other[1]), f"picks differ from the {name} layer"
            assert torch.equal(a[2], other[2]), f"weights differ from the {name} layer"
            _same(a[0], other[0], name)
    assert K.workspace_error(K.moe_workspace(g, 1, 8, 1, E, DEV)) == 0
