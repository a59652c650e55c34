"""GPU: the prefill path (expert-grouped dequant -> bf16 MFMA GEMMs) against
the oracle.

Routing and dispatch stay bit-exact; expert outputs and layer outputs are
held to tests/util tolerance against the float64 oracle (small shapes) or the
oracle's fp32 C restatement on sampled tokens (full Qwen3-235B shapes).
Router logits are skewed by a per-expert bias so expert loads are uneven and
heavy experts span several row tiles.
"""

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import pmoe_oracle as O
from tests.util import bits_to_bf16_tensor, check_close, expert_to_comps, fill_slab_gpu, slot_to_expert

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _k():
    from pagedmoe_amd import kernels
    return kernels


def _slab(spec, experts, extra=()):
    from pagedmoe_amd._lib import geom
    from pagedmoe_amd.slab import SlabStore
    g = geom(spec.hidden, spec.inter, spec.bits)
    allx = [experts[e] for e in range(spec.experts)] + list(extra)
    slab = SlabStore(g, len(allx), DEV)
    for i, ex in enumerate(allx):
        slab.write_expert(i, expert_to_comps(ex))
    return g, slab


def _x(rng, n, d):
    return O.bf16_round(rng.standard_normal((n, d), dtype=np.float32))


def test_prefill_path_is_selected():
    from pagedmoe_amd import _lib
    K = _k()
    g = _lib.geom(1024, 512, 4)
    # 512 tokens x top-4 over 32 experts = 2048 rows: the MFMA path
    slab = torch.zeros(32 * g.expert_bytes, dtype=torch.uint8, device=DEV)
    table = torch.arange(32, dtype=torch.int32, device=DEV)
    x = torch.zeros((512, 1024), dtype=torch.bfloat16, device=DEV)
    inds = torch.randint(0, 32, (512, 4), dtype=torch.int32, device=DEV)
    with _lib.KernelTimer() as kt:
        K.switch_glu(g, slab, table, 32, x, inds)
    torch.cuda.synchronize()
    assert "prefill_gateup" in kt.result and "prefill_down" in kt.result


@pytest.mark.parametrize("bits", [4, 6])
def test_prefill_moe_block_vs_oracle(bits):
    """D1024/E32/I512 top-4, 512 tokens (2048 rows), skewed routing."""
    K = _k()
    spec = O.LayerSpec(1024, 32, 512, 4, bits=bits)
    gw, experts, _, _, _ = O.make_layer(spec, seed=20 + bits)
    rng = np.random.default_rng(21)
    lb = rng.standard_normal(spec.experts, dtype=np.float32)
    xb = _x(rng, 512, spec.hidden)
    ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts, logit_bias=lb)
    counts = np.bincount(ref_i.reshape(-1), minlength=spec.experts)
    assert counts.max() > _tile_rows(512, 4, 32), "skew should give an expert several tiles"
    g, slab = _slab(spec, experts)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", spec.experts, spec.top_k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gw, DEV),
                               bits_to_bf16_tensor(xb, DEV),
                               logit_bias=torch.from_numpy(lb).to(DEV))
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out.float().cpu().numpy(), ref, f"prefill block {bits}-bit")


def test_prefill_switch_glu_seam_and_nonresident():
    """The seam at prefill size: y [N, K, D] per slot vs the oracle; an
    expert whose table entry is -1 gives exact zero rows."""
    K = _k()
    spec = O.LayerSpec(1024, 16, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=30)
    rng = np.random.default_rng(31)
    xb = _x(rng, 320, spec.hidden)
    inds = np.stack([rng.choice(spec.experts, 4, replace=False) for _ in range(320)]).astype(np.int32)
    g, slab = _slab(spec, experts)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    table[5] = -1
    y = K.switch_glu(g, slab.buf, table, spec.experts, bits_to_bf16_tensor(xb, DEV),
                     torch.from_numpy(inds).to(DEV)).float().cpu().numpy()
    assert (y[inds == 5] == 0).all()
    ref = O.switch_glu_f64(xb, inds, experts)
    mask = inds != 5
    check_close(y[mask], ref[mask], "prefill seam")


def test_prefill_switch_glu_unaligned_output_matches_aligned():
    """The down GEMM writes bf16 rows through LDS as 16-byte pieces when the
    output is 16-byte aligned and element by element otherwise: y at a
    2-byte offset (the element-wise path) equals the aligned result bit for
    bit, at 128-row tiles."""
    import ctypes
    from pagedmoe_amd import kernels as KM
    from pagedmoe_amd._lib import check, lib
    K = _k()
    spec = O.LayerSpec(1024, 16, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=32)
    rng = np.random.default_rng(33)
    n, k = 320, 4
    xb = _x(rng, n, spec.hidden)
    inds = torch.from_numpy(np.stack([rng.choice(spec.experts, k, replace=False)
                                      for _ in range(n)]).astype(np.int32)).to(DEV)
    assert _tile_rows(n, k, spec.experts) == 128
    g, slab = _slab(spec, experts)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    x = bits_to_bf16_tensor(xb, DEV)
    y_al = K.switch_glu(g, slab.buf, table, spec.experts, x, inds)
    big = torch.full((n * k * spec.hidden + 8,), float("nan"), dtype=torch.bfloat16, device=DEV)
    y_un = big[1:1 + n * k * spec.hidden]
    assert y_un.data_ptr() % 16 == 2
    ws = KM.moe_workspace(g, n, k, 0, spec.experts, x.device)
    check(lib().pmoe_switch_glu(ctypes.byref(g), KM._ptr(slab.buf), KM._table_ptr(table),
                                spec.experts, KM._ptr(x), KM._ptr(inds), n, k,
                                ctypes.c_void_p(y_un.data_ptr()), KM._ptr(ws), ws.numel(),
                                KM._stream()), "pmoe_switch_glu")
    torch.cuda.synchronize()
    assert torch.equal(y_al.reshape(-1).view(torch.int16), y_un.view(torch.int16))
    assert torch.isnan(big[0]) and torch.isnan(big[-7:]).all()


def test_prefill_sigmoid_shared_vs_oracle():
    """DeepSeek-style routing (sigmoid + bias, 8 groups / top-4, top-6,
    scale 2.5) with a shared expert: 384 tokens x 7 columns."""
    K = _k()
    spec = O.LayerSpec(1024, 64, 512, 6, scoring="sigmoid", n_group=8, topk_group=4,
                       routed_scale=2.5, shared=1)
    gw, experts, bias, sh, _ = O.make_layer(spec, seed=40)
    rng = np.random.default_rng(41)
    xb = _x(rng, 384, spec.hidden)
    ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts, bias=bias, shared=sh)
    g, slab = _slab(spec, experts, extra=sh)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("sigmoid", spec.experts, spec.top_k, True, 8, 4, 2.5)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gw, DEV),
                               bits_to_bf16_tensor(xb, DEV),
                               score_bias=torch.from_numpy(bias).to(DEV),
                               shared_slot=spec.experts)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out.float().cpu().numpy(), ref, "prefill sigmoid + shared")


def _small_layer(bits):
    """D1024/E64/I512 top-4 plus a shared expert, 256 tokens: 1,280 rows, ~16
    per routed expert, so the prefill cuts 32-row tiles and runs two blocks
    per CU.  Skewed routing gives some experts several tiles; the shared
    expert's 256 rows are eight."""
    spec = O.LayerSpec(1024, 64, 512, 4, bits=bits, shared=1)
    gw, experts, _, sh, _ = O.make_layer(spec, seed=70 + bits)
    rng = np.random.default_rng(71)
    lb = rng.standard_normal(spec.experts, dtype=np.float32) * np.float32(1.5)
    xb = _x(rng, 256, spec.hidden)
    return spec, gw, experts, sh, lb, xb


def _small_run(K, spec, gw, experts, sh, lb, xb, table_edit=None):
    g, slab = _slab(spec, experts, extra=sh)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    if table_edit is not None:
        table_edit(table)
    rc = K.route_cfg("softmax", spec.experts, spec.top_k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gw, DEV),
                               bits_to_bf16_tensor(xb, DEV), logit_bias=torch.from_numpy(lb).to(DEV),
                               shared_slot=spec.experts)
    return out, gi, gwt


@pytest.mark.parametrize("bits", [4, 6])
def test_prefill_small_tiles_vs_oracle(bits, monkeypatch):
    """The 32-row-tile form (chosen by rows per expert) against the float64
    oracle on every token, and bit-identical to the 128-row-tile form."""
    from pagedmoe_amd import _lib
    K = _k()
    spec, gw, experts, sh, lb, xb = _small_layer(bits)
    ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts, logit_bias=lb, shared=sh)
    counts = np.bincount(ref_i.reshape(-1), minlength=spec.experts)
    assert counts.max() > 64, "skew should give an expert three tiles"
    with _lib.KernelTimer() as kt:
        out, gi, gwt = _small_run(K, spec, gw, experts, sh, lb, xb)
    torch.cuda.synchronize()
    assert "prefill_gateup" in kt.result, "prefill path not taken"
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out.float().cpu().numpy(), ref, f"prefill small tiles {bits}-bit")
    monkeypatch.setenv("PMOE_PREFILL_SMALL", "0")
    big, _, _ = _small_run(K, spec, gw, experts, sh, lb, xb)
    assert torch.equal(out.view(torch.int16), big.view(torch.int16)), (
        f"forms differ: max |d| {(out.float() - big.float()).abs().max().item():.3e}")


def test_prefill_small_tiles_nonresident_and_forced_on_tall_tiles(monkeypatch):
    """An expert whose table entry is -1 gives exact zero rows in the
    32-row-tile form; that form pinned on for the skewed 512-token layer
    (experts of up to ~200 rows) matches the 128-row-tile form bit for
    bit."""
    K = _k()
    spec, gw, experts, sh, lb, xb = _small_layer(4)
    ids = O.softmax_topk(O.router_logits(xb, gw, lb), spec.top_k)[0]
    gone = int(np.bincount(ids.reshape(-1), minlength=spec.experts).argmax())

    def drop(table):
        table[gone] = -1

    out, gi, _ = _small_run(K, spec, gw, experts, sh, lb, xb, table_edit=drop)
    ref_i, ref_w = O.softmax_topk(O.router_logits(xb, gw, lb), spec.top_k)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    y = O.switch_glu_f64(xb, ref_i, experts)
    y[ref_i == gone] = 0.0
    ref = O.combine_f64(y, ref_w, O.expert_ffn_f64(O.bf16_to_f32(xb), sh[0]))
    check_close(out.float().cpu().numpy(), ref, "prefill small tiles, expert absent")
    spec2 = O.LayerSpec(1024, 32, 512, 4)
    gw2, experts2, _, _, _ = O.make_layer(spec2, seed=24)
    rng = np.random.default_rng(21)
    lb2 = rng.standard_normal(spec2.experts, dtype=np.float32)
    xb2 = _x(rng, 512, spec2.hidden)
    g2, slab2 = _slab(spec2, experts2)
    table2 = torch.arange(spec2.experts, dtype=torch.int32, device=DEV)
    rc2 = K.route_cfg("softmax", spec2.experts, spec2.top_k)
    outs = []
    for pin in ("1", "0"):
        monkeypatch.setenv("PMOE_PREFILL_SMALL", pin)
        o, _, _ = K.moe_block(g2, rc2, slab2.buf, table2, bits_to_bf16_tensor(gw2, DEV),
                              bits_to_bf16_tensor(xb2, DEV), logit_bias=torch.from_numpy(lb2).to(DEV))
        outs.append(o)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def _tile_rows(n, kk, n_experts):
    from pagedmoe_amd import _lib
    return int(_lib.lib().pmoe_prefill_tile_rows(n, kk, n_experts))


def _tile_boundary_tokens(inds, tile_m):
    """Tokens whose rows sit at the row-tile edges of the heaviest expert:
    the first and last row of every row tile, and the partial last tile's
    last row.  The dispatch orders an expert's rows by flat index
    (token * K + slot), so the expert's p-th row is its p-th occurrence in
    the flat routing."""
    flat = inds.reshape(-1)
    counts = np.bincount(flat, minlength=int(flat.max()) + 1)
    heavy = int(np.argmax(counts))
    rows = np.flatnonzero(flat == heavy)
    pos = {0, len(rows) - 1}
    for t0 in range(0, len(rows), tile_m):
        pos.update({t0, min(t0 + tile_m - 1, len(rows) - 1)})
    k = inds.shape[1]
    return sorted({int(rows[p]) // k for p in pos})


def test_prefill_qwen3_235b_2048_tokens_sampled():
    """Full prefill shape: D4096/E128/I1536 top-8 4-bit, 2048 tokens with
    router logits skewed by a N(0,1) per-expert bias.  Routing of every token
    bit-exact (C oracle router); the layer output of the tokens at the
    heaviest expert's row-tile edges (first and last row of each row tile,
    the partial last tile) and of 6 random tokens within tolerance of the
    fp32 C restatement of the experts."""
    K = _k()
    from pagedmoe_amd._lib import geom
    from pagedmoe_amd.slab import SlabStore
    D, E, I, k = 4096, 128, 1536, 8
    g = geom(D, I, 4)
    slab = SlabStore(g, E, DEV)
    fill_slab_gpu(slab, range(E), seed=50)
    rng = np.random.default_rng(51)
    gwb = O.bf16_round(rng.standard_normal((E, D), dtype=np.float32) * np.float32(0.02))
    lb = rng.standard_normal(E, dtype=np.float32)
    xb = _x(rng, 2048, D)
    table = torch.arange(E, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", E, k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV),
                               logit_bias=torch.from_numpy(lb).to(DEV))
    logits = C.router_logits(xb, gwb, lb)
    ref_i, ref_w = O.softmax_topk(logits, k)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    out = out.float().cpu().numpy()
    sample = (_tile_boundary_tokens(ref_i, _tile_rows(2048, k, E))
              + [int(t) for t in rng.choice(2048, 6, replace=False)])
    cache = {}
    for t in sample:
        x = O.bf16_to_f32(xb[t])
        acc = np.zeros(D, np.float64)
        for j in range(k):
            e = int(ref_i[t, j])
            if e not in cache:
                cache[e] = slot_to_expert(slab, e)
            acc += np.float64(ref_w[t, j]) * C.expert_ffn(cache[e], x, D, I, 4).astype(np.float64)
        check_close(out[t], acc, f"235B prefill token {t}")


def test_prefill_qwen3_next_1024_tokens_sampled():
    """Full Qwen3-Next prefill shape: D2048/E512/I512 top-10 6-bit plus a
    sigmoid-gated shared expert, 1024 tokens (10,240 routed rows over 512
    experts, ~20 per expert: one partial tile each).  Routing of every token
    bit-exact (C oracle router); the layer output of the tokens at the
    heaviest expert's tile edges and of 6 random tokens within tolerance of
    the fp32 C restatement of the experts."""
    K = _k()
    from pagedmoe_amd._lib import geom
    from pagedmoe_amd.slab import SlabStore
    D, E, I, k = 2048, 512, 512, 10
    g = geom(D, I, 6)
    slab = SlabStore(g, E + 1, DEV)
    fill_slab_gpu(slab, range(E + 1), seed=60)
    rng = np.random.default_rng(61)
    gwb = O.bf16_round(rng.standard_normal((E, D), dtype=np.float32) * np.float32(0.02))
    sgb = O.bf16_round(rng.standard_normal((1, D), dtype=np.float32) * np.float32(0.02))
    xb = _x(rng, 1024, D)
    table = torch.arange(E, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", E, k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV), shared_slot=E,
                               shared_gate=bits_to_bf16_tensor(sgb, DEV))
    ref_i, ref_w = O.softmax_topk(C.router_logits(xb, gwb), k)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    out = out.float().cpu().numpy()
    gate_logit = C.router_logits(xb, sgb)[:, 0].astype(np.float64)
    shared = slot_to_expert(slab, E)
    sample = (_tile_boundary_tokens(ref_i, _tile_rows(1024, k + 1, E))
              + [int(t) for t in rng.choice(1024, 6, replace=False)])
    cache = {}
    for t in sample:
        x = O.bf16_to_f32(xb[t])
        acc = np.zeros(D, np.float64)
        for j in range(k):
            e = int(ref_i[t, j])
            if e not in cache:
                cache[e] = slot_to_expert(slab, e)
            acc += np.float64(ref_w[t, j]) * C.expert_ffn(cache[e], x, D, I, 6).astype(np.float64)
        gate = 1.0 / (1.0 + np.exp(-gate_logit[t]))
        acc += gate * C.expert_ffn(shared, x, D, I, 6).astype(np.float64)
        check_close(out[t], acc, f"qwen3-next prefill token {t}")
