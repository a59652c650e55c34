"""GPU: the one-launch decode layer (decode_fused.hip).

The fused kernel runs the same GEMV arithmetic and combine order as the
three-launch decode (router, gate/up, down+combine), so its outputs must be
bit-identical to that path on the same inputs; routing must equal the oracle
bit for bit.  The grid-barrier counters in the workspace header must be back
at zero after every call and the launch epoch must count the grid-wide calls
(checked through repeated calls, batch-size changes and HIP-graph replays);
the sticky error word must stay 0.

One token with top-8 softmax routing and no shared expert takes the
expert-per-XCD form (pick x streamed by block group x, logits and h
exchanged as tagged words, the last of 8 groups combining each down tile).
Its counters only grow, by exact amounts per call (blocks-per-group on each
group's launch counter, 8 on each down-tile counter), which is how these
tests tell that it ran; its outputs must equal the grid-wide launch's and
the three-launch path's bit for bit, also under HIP-graph replay (where the
dispatcher starts the grid mid-cycle over the XCDs).
"""

import os

import numpy as np
import pytest
import torch

from oracle import pmoe_oracle as O
from tests.util import bits_to_bf16_tensor, check_close, fill_slab_gpu, slot_to_expert

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _fused_on(monkeypatch):
    monkeypatch.setenv("PMOE_DECODE_FUSED", "1")


def _k():
    from pagedmoe_amd import kernels
    return kernels


class _Layer:
    """Random resident layer of a given shape on the GPU."""

    def __init__(self, hidden, experts, inter, top_k, bits=4, scoring="softmax", shared=False,
                 shared_gate=False, seed=0, n_group=1, topk_group=1, scale=1.0):
        from pagedmoe_amd._lib import geom
        from pagedmoe_amd.slab import SlabStore
        K = _k()
        self.g = geom(hidden, inter, bits)
        n_slots = experts + (1 if shared else 0)
        self.slab = SlabStore(self.g, n_slots, DEV)
        fill_slab_gpu(self.slab, range(n_slots), seed=seed)
        rng = np.random.default_rng(seed)
        self.gwb = O.bf16_round(rng.standard_normal((experts, hidden), dtype=np.float32)
                                * np.float32(0.02))
        self.gate = bits_to_bf16_tensor(self.gwb, DEV)
        self.table = torch.arange(experts, dtype=torch.int32, device=DEV)
        self.rc = K.route_cfg(scoring, experts, top_k, True, n_group, topk_group, scale)
        self.bias = None
        if scoring == "sigmoid":
            b = (rng.standard_normal(experts, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
            self.bias = torch.from_numpy(b).to(DEV)
        self.shared_slot = experts if shared else -1
        self.sgate = None
        if shared_gate:
            sgb = O.bf16_round(rng.standard_normal((1, hidden), dtype=np.float32) * np.float32(0.02))
            self.sgate = bits_to_bf16_tensor(sgb, DEV)
        self.hidden = hidden
        self.experts = experts

    def x(self, n, seed):
        rng = np.random.default_rng(seed)
        return bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((n, self.hidden),
                                                                    dtype=np.float32)), DEV)

    def run(self, x, ws=None, out=None, inds=None, weights=None):
        return _k().moe_block(self.g, self.rc, self.slab.buf, self.table, self.gate, x,
                              score_bias=self.bias, shared_slot=self.shared_slot,
                              shared_gate=self.sgate, ws=ws, out=out, inds=inds, weights=weights)


def _run_path(layer, x, fused, ws=None, xcd=True):
    saved = {v: os.environ.get(v) for v in ("PMOE_DECODE_FUSED", "PMOE_DECODE_XCD")}
    os.environ["PMOE_DECODE_FUSED"] = "1" if fused else "0"
    os.environ["PMOE_DECODE_XCD"] = "1" if xcd else "0"
    try:
        out, inds, wts = layer.run(x, ws=ws)
        torch.cuda.synchronize()
    finally:
        for v, old in saved.items():
            if old is None:
                del os.environ[v]
            else:
                os.environ[v] = old
    return out.clone(), inds.clone(), wts.clone()


def _fused_launches(layer, x):
    from pagedmoe_amd._lib import KernelTimer
    with KernelTimer() as kt:
        layer.run(x)
    torch.cuda.synchronize()
    return kt.result


# Group arrival counters of the two grid barriers: 2 x 32 lines of 128 bytes
# after the 256-byte header and the 512 per-block flag lines.
GROUP_OFFSET = 256 + 512 * 128
SYNC_BYTES = GROUP_OFFSET + 2 * 32 * 128


def _assert_group_counters_reset(ws):
    grp = ws[GROUP_OFFSET:SYNC_BYTES].cpu().view(torch.int32).numpy()
    assert not grp.any(), f"group arrival counters not reset: {np.nonzero(grp)}"


# Expert-per-XCD launch: 8 group launch counters (128 bytes apart), then
# 1024 down-tile counters (64 bytes apart).
XCD_OFFSET = SYNC_BYTES
TILE_OFFSET = XCD_OFFSET + 8 * 128


def _xcd_counters(ws):
    xc = ws[XCD_OFFSET:TILE_OFFSET].cpu().view(torch.int32).numpy()[::32]
    tc = ws[TILE_OFFSET:TILE_OFFSET + 1024 * 64].cpu().view(torch.int32).numpy()[::16]
    return xc, tc


def _assert_xcd_calls(ws, calls, hidden=None):
    """The expert-per-XCD launch ran exactly `calls` times on ws: every
    group's launch counter holds blocks-per-group per call, and each down
    tile (8 or 16 rows) covering `hidden` counted 8 arrivals per call."""
    per_xcd = torch.cuda.get_device_properties(0).multi_processor_count // 8
    xc, tc = _xcd_counters(ws)
    assert (xc == per_xcd * calls).all(), f"group counters {xc} after {calls} calls"
    used = int(np.count_nonzero(tc))
    assert (tc[:used] == 8 * calls).all() and not tc[used:].any(), f"tile counters {tc[:used + 2]}"
    if calls and hidden:
        assert used in ((hidden + 7) // 8, (hidden + 15) // 16), f"{used} tiles for {hidden} rows"


CASES = {
    # hidden, experts, inter, top_k, bits, scoring, shared, shared_gate, n_group, topk_group, scale
    "qwen3-235b": (4096, 128, 1536, 8, 4, "softmax", False, False, 1, 1, 1.0),
    "deepseek-shapes": (7168, 64, 2048, 8, 4, "sigmoid", True, False, 8, 4, 2.5),
    "qwen3-next-6bit": (2048, 512, 512, 10, 6, "softmax", True, True, 1, 1, 1.0),
    "tiny": (1024, 32, 512, 4, 4, "softmax", False, False, 1, 1, 1.0),
    # single-token rank routing with the shared-expert column and its gate
    "tiny-shared-gate": (1024, 96, 512, 6, 4, "softmax", True, True, 1, 1, 1.0),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("n", [1, 8])
def test_fused_matches_three_launch_bit_exact(name, n):
    h, e, i, k, bits, sc, shared, sg, ng, tg, scale = CASES[name]
    print(f"[fused] case {name} n={n}", flush=True)
    layer = _Layer(h, e, i, k, bits, sc, shared, sg, seed=21, n_group=ng, topk_group=tg,
                   scale=scale)
    x = layer.x(n, seed=100 + n)
    launched = _fused_launches(layer, x)
    assert any(kn in launched for kn in ("decode_fused", "decode_xcd", "experts_xcd")), (
        "fused path not taken")
    a = _run_path(layer, x, fused=True)
    b = _run_path(layer, x, fused=False)
    assert torch.equal(a[1], b[1]), "routing indices differ"
    assert torch.equal(a[2], b[2]), "routing weights differ"
    assert torch.equal(a[0].view(torch.int16), b[0].view(torch.int16)), (
        f"outputs differ: max |d| {(a[0].float() - b[0].float()).abs().max().item():.3e}")
    ws = _k().moe_workspace(layer.g, n, k, int(shared), e, DEV)
    assert _k().workspace_error(ws) == 0


def test_fused_qwen3_235b_vs_oracle_and_reuse_across_batches():
    """One workspace, batch sizes 1 -> 8 -> 3 -> 1: every call equals the
    oracle routing and the float64 reference within tolerance."""
    K = _k()
    layer = _Layer(4096, 128, 1536, 8, seed=5)
    ws = K.moe_workspace(layer.g, 8, 8, 0, 128, DEV, fresh=True)
    for step, n in enumerate((1, 8, 3, 1)):
        print(f"[fused] reuse step {step} n={n}", flush=True)
        x = layer.x(n, seed=300 + step)
        out, gi, gw = layer.run(x, ws=ws)
        xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
        ref_i, ref_w = O.softmax_topk(O.router_logits(xb, layer.gwb), 8)
        assert np.array_equal(gi.cpu().numpy(), ref_i)
        assert np.array_equal(gw.cpu().numpy(), ref_w)
        used = sorted(set(ref_i.reshape(-1).tolist()))
        experts = {e: slot_to_expert(layer.slab, e) for e in used}
        ref = O.combine_f64(O.switch_glu_f64(xb, ref_i, experts), ref_w)
        check_close(out.float().cpu().numpy(), ref, f"fused reuse n={n}")
    header = ws[:16].cpu().view(torch.int32).numpy()
    assert header[0] == 0 and header[1] == 0, f"barrier counters not reset: {header}"
    assert header[2] == 2, f"launch epoch {header[2]} after 2 grid-wide calls"
    assert header[3] == 0, "barrier timeout flagged"
    _assert_group_counters_reset(ws)
    _assert_xcd_calls(ws, 2, 4096)    # the two single-token calls


def test_fused_graph_replays_match_eager():
    """A HIP graph of four layer steps (fused launches), replayed with fresh
    inputs and eager work in between, equals eager runs bit for bit."""
    K = _k()
    layer = _Layer(4096, 128, 1536, 8, seed=7)
    n, steps = 1, 4
    ws = K.moe_workspace(layer.g, n, 8, 0, 128, DEV, fresh=True)
    xs = torch.empty((steps, n, 4096), dtype=torch.bfloat16, device=DEV)
    outs = torch.empty((steps, n, 4096), dtype=torch.bfloat16, device=DEV)
    inds = torch.empty((steps, n, 8), dtype=torch.int32, device=DEV)
    wts = torch.empty((steps, n, 8), dtype=torch.float32, device=DEV)

    def seq():
        for s in range(steps):
            layer.run(xs[s], ws=ws, out=outs[s], inds=inds[s], weights=wts[s])

    for s in range(steps):
        xs[s].copy_(layer.x(n, seed=400 + s))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        seq()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        seq()
    torch.cuda.synchronize()
    for rep in range(4):
        print(f"[fused] graph replay {rep}", flush=True)
        for s in range(steps):
            xs[s].copy_(layer.x(n, seed=500 + 10 * rep + s))
        graph.replay()
        torch.cuda.synchronize()
        got = outs.clone(), inds.clone(), wts.clone()
        ref_ws = K.moe_workspace(layer.g, n, 8, 0, 128, DEV)
        for s in range(steps):
            eo, ei, ew = layer.run(xs[s].clone(), ws=ref_ws)
            torch.cuda.synchronize()
            assert torch.equal(ei, got[1][s]) and torch.equal(ew, got[2][s])
            assert torch.equal(eo.view(torch.int16), got[0][s].view(torch.int16)), \
                f"replay {rep} step {s} differs from eager"
    assert K.workspace_error(ws) == 0
    header = ws[:16].cpu().view(torch.int32).numpy()
    assert header[0] == 0 and header[1] == 0, f"barrier counters not reset: {header}"
    _assert_group_counters_reset(ws)
    _assert_xcd_calls(ws, steps * 5, 4096)   # eager warm-up + 4 replays


XCD_CASES = {
    # hidden, experts, inter, bits
    "qwen3-235b": (4096, 128, 1536, 4),
    "qwen3-30b": (2048, 128, 768, 4),
    "small": (1024, 64, 512, 4),
    "small-6bit": (1024, 64, 512, 6),
}


@pytest.mark.parametrize("name", sorted(XCD_CASES))
def test_xcd_split_matches_grid_wide_and_three_launch(name):
    """Expert-per-XCD launch against the grid-wide launch and the
    three-launch path on the same inputs, with every third expert absent
    from the slot table (exact zero rows): routing and outputs bit for bit,
    three calls on one workspace, counters advanced exactly."""
    K = _k()
    h, e, i, bits = XCD_CASES[name]
    print(f"[xcd] case {name}", flush=True)
    layer = _Layer(h, e, i, 8, bits, seed=61)
    layer.table[::3] = -1
    ws_x = K.moe_workspace(layer.g, 1, 8, 0, e, DEV, fresh=True)
    ws_g = K.moe_workspace(layer.g, 1, 8, 0, e, DEV, fresh=True)
    absent_hit = False
    for call in range(3):
        x = layer.x(1, seed=610 + call)
        a = _run_path(layer, x, fused=True, ws=ws_x, xcd=True)
        b = _run_path(layer, x, fused=True, ws=ws_g, xcd=False)
        c = _run_path(layer, x, fused=False)
        for other, what in ((b, "grid-wide launch"), (c, "three-launch path")):
            assert torch.equal(a[1], other[1]), f"call {call}: indices differ from the {what}"
            assert torch.equal(a[2], other[2]), f"call {call}: weights differ from the {what}"
            assert torch.equal(a[0].view(torch.int16), other[0].view(torch.int16)), (
                f"call {call}: outputs differ from the {what}: max |d| "
                f"{(a[0].float() - other[0].float()).abs().max().item():.3e}")
        absent_hit |= bool((a[1] % 3 == 0).any())
    assert absent_hit, "no absent expert was picked: the zero-row case went untested"
    _assert_xcd_calls(ws_x, 3, h)
    _assert_xcd_calls(ws_g, 0)
    assert K.workspace_error(ws_x) == 0 and K.workspace_error(ws_g) == 0


@pytest.mark.parametrize("n", [1, 2])
def test_fused_routing_exact_ties_lower_id_first(n):
    """Pairs of identical router rows give exactly tied logits: the one-launch
    routing (rank counts for one token, the wave top-k for more) must pick
    and order them as the three-launch routing and the oracle do -- value
    descending, lower expert id first."""
    h, e, i, k = 1024, 64, 512, 8
    print(f"[fused] exact ties n={n}", flush=True)
    layer = _Layer(h, e, i, k, seed=33)
    layer.gwb[1::2] = layer.gwb[0::2]  # expert 2j+1 duplicates expert 2j
    layer.gate = bits_to_bf16_tensor(layer.gwb, DEV)
    x = layer.x(n, seed=7)
    a = _run_path(layer, x, fused=True)
    b = _run_path(layer, x, fused=False)
    assert torch.equal(a[1], b[1]), "routing indices differ"
    assert torch.equal(a[2], b[2]), "routing weights differ"
    assert torch.equal(a[0].view(torch.int16), b[0].view(torch.int16)), "outputs differ"
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    lg = O.router_logits(xb, layer.gwb)
    ref_i, ref_w = O.softmax_topk(lg, k)
    inds = a[1].cpu().numpy()
    assert np.array_equal(inds, ref_i), f"{inds} vs oracle {ref_i}"
    assert np.array_equal(a[2].cpu().numpy(), ref_w)
    tied = lg[:, 0::2] == lg[:, 1::2]
    assert tied.all(), "duplicated router rows must give exactly tied logits"
    # every picked odd id sits right after its even twin
    for row in inds:
        for j, v in enumerate(row):
            if v % 2 == 1:
                assert j > 0 and row[j - 1] == v - 1, f"tie order broken: {row}"


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n", [1, 3, 8])
def test_routing_512_experts_vs_oracle(n, fused):
    """Top-10 of 512 softmax-renormalised experts (eight logits per lane in
    the wave top-k) against the oracle: indices and weights bit-exact, on
    both decode paths."""
    h, e, i, k = 1024, 512, 512, 10
    print(f"[fused] 512-expert routing n={n} fused={fused}", flush=True)
    layer = _Layer(h, e, i, k, seed=44)
    x = layer.x(n, seed=900 + n)
    _, inds, wts = _run_path(layer, x, fused=fused)
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    ref_i, ref_w = O.softmax_topk(O.router_logits(xb, layer.gwb), k)
    assert np.array_equal(inds.cpu().numpy(), ref_i)
    assert np.array_equal(wts.cpu().numpy(), ref_w)


@pytest.mark.parametrize("xcd", [True, False])
def test_barrier_timeout_poisons_output_and_is_reported(xcd, monkeypatch):
    """A barrier wait that gives up (forced from the host with a one-tick
    spin limit on the kernel's own bounded wait, so every block still exits
    normally) sets error bit 0, leaves NaN in the layer output instead of a
    plausible wrong answer, and raises PmoeError at the next host sync point,
    which also re-initialises the workspace -- for the expert-per-XCD launch
    and the grid-wide one."""
    from pagedmoe_amd._lib import PmoeError
    K = _k()
    monkeypatch.setenv("PMOE_DECODE_XCD", "1" if xcd else "0")
    layer = _Layer(4096, 128, 1536, 8, seed=9)
    ws = K.moe_workspace(layer.g, 1, 8, 0, 128, DEV)   # the cached one the sync points read
    x = layer.x(1, seed=900)
    good, _, _ = layer.run(x, ws=ws)
    torch.cuda.synchronize()
    assert K.workspace_error(ws) == 0
    print(f"[fused] barrier spin limit 1 tick, xcd={xcd}", flush=True)
    K.set_barrier_spin(1)
    try:
        bad, _, _ = layer.run(x, ws=ws)
        torch.cuda.synchronize()
    finally:
        K.set_barrier_spin(0)
    assert K.workspace_error(ws) & 1
    assert torch.isnan(bad.float()).all(), "a timed-out layer wrote finite outputs"
    with pytest.raises(PmoeError, match="timed out"):
        K.check_workspace_errors()
    again, _, _ = layer.run(x, ws=ws)
    torch.cuda.synchronize()
    assert K.workspace_error(ws) == 0
    assert torch.equal(again.view(torch.int16), good.view(torch.int16))


def test_graph_on_cached_workspace_survives_a_larger_call(monkeypatch):
    """A graph captured over the cached workspace keeps its raw pointer; a
    later, larger eager call (a prefill) replaces the cached workspace but
    must not free the old one, so replays stay bit-identical to eager runs.
    Growing the workspace during a capture is refused."""
    from pagedmoe_amd._lib import PmoeError
    K = _k()
    dev = torch.device(DEV).index or 0
    old = K._MOE_WS.pop(dev, None)
    if old is not None:
        K._RETIRED["MoE"].append(old)
    layer = _Layer(1024, 32, 512, 4, seed=11)
    out = torch.empty((1, 1024), dtype=torch.bfloat16, device=DEV)
    inds = torch.empty((1, 4), dtype=torch.int32, device=DEV)
    wts = torch.empty((1, 4), dtype=torch.float32, device=DEV)
    x = torch.empty((1, 1024), dtype=torch.bfloat16, device=DEV)
    x.copy_(layer.x(1, seed=1100))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.run(x, out=out, inds=inds, weights=wts)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    captured = K._MOE_WS[dev].data_ptr()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer.run(x, out=out, inds=inds, weights=wts)
    torch.cuda.synchronize()
    big, _, _ = layer.run(layer.x(512, seed=1101))      # grows the cached workspace
    torch.cuda.synchronize()
    assert K._MOE_WS[dev].data_ptr() != captured
    assert any(b.data_ptr() == captured for b in K._RETIRED["MoE"])
    filler = torch.full((64 << 20,), 7, dtype=torch.uint8, device=DEV)  # reuses freed memory
    for rep in range(3):
        x.copy_(layer.x(1, seed=1110 + rep))
        graph.replay()
        torch.cuda.synchronize()
        ref, ri, rw = layer.run(x.clone())
        torch.cuda.synchronize()
        assert torch.equal(ri, inds) and torch.equal(rw, wts)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), rep
    del filler, big
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(PmoeError, match="during graph capture"):
        K.moe_workspace(layer.g, 4096, 4, 0, 32, DEV)


def test_split_group_is_reported_at_once(monkeypatch):
    """The expert-per-XCD launch checks that each block group shares one
    XCD (its h words travel through that XCD's L2).  Forced from the host
    (block 0 reports another XCD; every block still exits normally): error
    bit 1 is set and the layer output is NaN within the launch -- no block
    waits out the 0.5 s spin limit -- PmoeError is raised at the next sync
    point, and the next call is bit-exact again."""
    import time

    from pagedmoe_amd._lib import PmoeError
    K = _k()
    monkeypatch.setenv("PMOE_DECODE_XCD", "1")
    layer = _Layer(4096, 128, 1536, 8, seed=9)
    ws = K.moe_workspace(layer.g, 1, 8, 0, 128, DEV)
    x = layer.x(1, seed=901)
    assert "decode_xcd" in _fused_launches(layer, x)
    good, _, _ = layer.run(x, ws=ws)
    torch.cuda.synchronize()
    assert K.workspace_error(ws) == 0
    print("[fused] split probe on", flush=True)
    K.set_split_probe(True)
    try:
        t0 = time.perf_counter()
        bad, _, _ = layer.run(x, ws=ws)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    finally:
        K.set_split_probe(False)
    assert K.workspace_error(ws) & 2
    assert torch.isnan(bad.float()).any(), "a split group wrote only finite outputs"
    assert dt < 0.2, f"the split launch took {dt:.3f} s: a poll waited out its limit"
    with pytest.raises(PmoeError, match="different XCDs"):
        K.check_workspace_errors()
    again, _, _ = layer.run(x, ws=ws)
    torch.cuda.synchronize()
    assert K.workspace_error(ws) == 0
    assert torch.equal(again.view(torch.int16), good.view(torch.int16))
