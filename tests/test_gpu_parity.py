"""GPU parity: HIP kernels through the C ABI vs the CPU oracle.

Bit-exact: router logits, routing indices and weights, dispatch permutation,
quantize/dequantize.  Within tolerance (tests/util.check_close): expert
outputs and layer outputs against the float64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import pmoe_oracle as O
from tests.util import (bf16_tensor_bits, bits_to_bf16_tensor, check_close, expert_to_comps,
                        fill_slab_gpu, slot_to_expert)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _k():
    from pagedmoe_amd import kernels
    return kernels


def _x_bits(rng, n, d):
    return O.bf16_round(rng.standard_normal((n, d), dtype=np.float32))


@pytest.mark.parametrize("n,d,e", [(64, 1024, 32), (1, 4096, 128), (8, 4096, 128),
                                   (200, 4096, 128), (3, 7168, 384), (8, 2048, 512),
                                   (517, 4096, 128), (1000, 2048, 513)])
def test_router_logits_bit_exact(n, d, e):
    K = _k()
    rng = np.random.default_rng(n * 7 + e)
    xb = _x_bits(rng, n, d)
    wb = O.bf16_round(rng.standard_normal((e, d), dtype=np.float32) * np.float32(0.02))
    bias = rng.standard_normal(e, dtype=np.float32)
    ref = O.router_logits(xb, wb, bias)
    got = K.router_logits(bits_to_bf16_tensor(xb, DEV), bits_to_bf16_tensor(wb, DEV),
                          torch.from_numpy(bias).to(DEV)).cpu().numpy()
    assert np.array_equal(got, ref), f"max |d| {np.abs(got - ref).max()}"


@pytest.mark.parametrize("n,e,k,norm", [(64, 32, 4, True), (8, 128, 8, True), (33, 512, 10, True),
                                        (5, 128, 8, False), (2, 7, 7, True)])
def test_softmax_topk_bit_exact(n, e, k, norm):
    K = _k()
    rng = np.random.default_rng(e + k)
    logits = rng.standard_normal((n, e), dtype=np.float32)
    logits[0, :3] = logits[0, 3]          # ties -> lower id first
    ref_i, ref_w = O.softmax_topk(logits, k, norm)
    gi, gw = K.route_softmax_topk(torch.from_numpy(logits).to(DEV), k, norm)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gw.cpu().numpy(), ref_w)


@pytest.mark.parametrize("n,e,ng,tg,k,scale", [(1, 384, 8, 4, 8, 2.5), (16, 256, 8, 4, 8, 2.5),
                                               (4, 64, 1, 1, 6, 1.0), (3, 96, 4, 4, 8, 1.5),
                                               (1, 64, 1, 1, 6, 1.0), (1, 384, 1, 1, 8, 2.5),
                                               (1, 256, 8, 2, 8, 2.5), (1, 96, 4, 4, 8, 1.5)])
def test_sigmoid_group_topk_bit_exact(n, e, ng, tg, k, scale):
    K = _k()
    rng = np.random.default_rng(e + n)
    logits = rng.standard_normal((n, e), dtype=np.float32)
    bias = (rng.standard_normal(e, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    ref_i, ref_w = O.sigmoid_group_topk(logits, bias, ng, tg, k, True, scale)
    gi, gw = K.route_sigmoid_group_topk(torch.from_numpy(logits).to(DEV),
                                        torch.from_numpy(bias).to(DEV), ng, tg, k, True, scale)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gw.cpu().numpy(), ref_w)


@pytest.mark.parametrize("ng,tg", [(8, 4), (1, 1)])
def test_sigmoid_one_token_ties_bit_exact(ng, tg):
    """One token (the block-parallel routing): equal biased scores inside a
    group, across groups and at a group's top two, a group score tie, and a
    kept group whose scores are all negative (the masked experts' zeros
    then win) -- lower id first among equals, as the oracle."""
    K = _k()
    e, k = 384, 8
    rng = np.random.default_rng(7)
    for case in range(4):
        logits = rng.standard_normal((1, e), dtype=np.float32)
        bias = (rng.standard_normal(e, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
        if case == 0:    # equal scores: 3 in group 0, 2 more in groups 5 and 7
            for i in (3, 9, 17, 5 * 48 + 1, 7 * 48 + 40):
                logits[0, i], bias[i] = np.float32(2.5), np.float32(0.3)
        elif case == 1:  # two groups with the same top two (same group score)
            for g, off in ((2, 0), (6, 0)):
                logits[0, g * 48 + 10 + off], bias[g * 48 + 10 + off] = np.float32(3.0), np.float32(0.2)
                logits[0, g * 48 + 20 + off], bias[g * 48 + 20 + off] = np.float32(2.0), np.float32(0.2)
        elif case == 2:  # a group's maximum repeated (counts twice in its score)
            for i in (4 * 48 + 1, 4 * 48 + 2):
                logits[0, i], bias[i] = np.float32(4.0), np.float32(0.5)
        else:            # scores below zero: masked experts (0.0) outrank kept ones
            bias[:] = np.float32(-2.0)
        ref_i, ref_w = O.sigmoid_group_topk(logits, bias, ng, tg, k, True, 2.5)
        gi, gw = K.route_sigmoid_group_topk(torch.from_numpy(logits).to(DEV),
                                            torch.from_numpy(bias).to(DEV), ng, tg, k, True, 2.5)
        assert np.array_equal(gi.cpu().numpy(), ref_i), (case, gi.cpu().numpy(), ref_i)
        assert np.array_equal(gw.cpu().numpy(), ref_w), case


@pytest.mark.parametrize("rows,e", [(0, 8), (1, 8), (64, 128), (1000, 32), (1024, 512),
                                    (16384, 128), (10240, 513), (5000, 3)])
def test_dispatch_bit_exact(rows, e):
    K = _k()
    rng = np.random.default_rng(rows + e)
    ids = rng.integers(0, e, size=rows).astype(np.int32)
    if rows > 10:
        ids[: rows // 3] = e - 1        # a heavy expert
    ref = O.dispatch(ids, e)
    got = K.dispatch(torch.from_numpy(ids).to(DEV), e)
    assert np.array_equal(got["order"].cpu().numpy(), ref.order)
    assert np.array_equal(got["counts"].cpu().numpy(), ref.counts)
    assert np.array_equal(got["offsets"].cpu().numpy(), ref.offsets)
    assert np.array_equal(got["inv"].cpu().numpy(), ref.inv)
    na = int(got["n_active"].item())
    assert na == len(ref.active)
    assert np.array_equal(got["active"].cpu().numpy()[:na], ref.active)


def test_dispatch_drops_out_of_range_ids():
    K = _k()
    ids = np.array([3, 9, -1, 3, 0], np.int32)
    got = K.dispatch(torch.from_numpy(ids).to(DEV), 4)
    inv = got["inv"].cpu().numpy()
    assert inv[1] == -1 and inv[2] == -1
    assert got["counts"].cpu().numpy().tolist() == [1, 0, 0, 2]
    assert got["order"].cpu().numpy()[:3].tolist() == [4, 0, 3]


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("rows,cols", [(16, 64), (96, 1024), (512, 4096)])
def test_quantize_dequant_bit_exact(bits, rows, cols):
    K = _k()
    rng = np.random.default_rng(rows + cols + bits)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    w[0, :64] = 0.125                      # constant group -> scale guard
    ref = O.quantize(w, bits)
    q, s, b = K.quantize(torch.from_numpy(w).to(DEV), bits)
    assert np.array_equal(q.cpu().numpy().view(np.uint32), ref.weight)
    assert np.array_equal(bf16_tensor_bits(s), ref.scales)
    assert np.array_equal(bf16_tensor_bits(b), ref.biases)
    deq = K.dequant(q, s, b, bits)
    assert np.array_equal(bf16_tensor_bits(deq), O.dequant_bf16(ref))


def _slab_from_experts(experts, spec, extra=()):
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd._lib import geom
    g = geom(spec.hidden, spec.inter, spec.bits)
    allx = list(experts) + list(extra)
    slab = SlabStore(g, len(allx), DEV)
    for i, ex in enumerate(allx):
        slab.write_expert(i, expert_to_comps(ex))
    return g, slab


def test_switch_glu_tiny_vs_oracle():
    """Config 1 shapes (D1024, E32, I512, top-4, 4-bit g64), N=64, seed 0."""
    K = _k()
    spec = O.LayerSpec(1024, 32, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=0)
    rng = np.random.default_rng(0)
    xb = _x_bits(rng, 64, spec.hidden)
    logits = O.router_logits(xb, gw)
    inds, _ = O.softmax_topk(logits, spec.top_k)
    g, slab = _slab_from_experts([experts[e] for e in range(spec.experts)], spec)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    y = K.switch_glu(g, slab.buf, table, spec.experts, bits_to_bf16_tensor(xb, DEV),
                     torch.from_numpy(inds).to(DEV))
    ref = O.switch_glu_f64(xb, inds, experts)
    check_close(y.float().cpu().numpy(), ref, "switch_glu tiny")


@pytest.mark.parametrize("bits", [4, 6])
def test_moe_block_tiny_vs_oracle(bits):
    K = _k()
    spec = O.LayerSpec(1024, 32, 512, 4, bits=bits)
    gw, experts, _, _, _ = O.make_layer(spec, seed=1)
    rng = np.random.default_rng(1)
    xb = _x_bits(rng, 64, spec.hidden)
    ref_i, ref_w, _, ref_out = O.moe_layer_f64(spec, xb, gw, experts)
    g, slab = _slab_from_experts([experts[e] for e in range(spec.experts)], spec)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", spec.experts, spec.top_k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gw, DEV),
                               bits_to_bf16_tensor(xb, DEV))
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out.float().cpu().numpy(), ref_out, "moe_block tiny")


@pytest.mark.parametrize("n", [1, 8])
def test_qwen3_235b_decode_vs_oracle(n):
    """Config 2 shapes (D4096, E128, I1536, top-8, 4-bit), all experts resident."""
    K = _k()
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd._lib import geom
    spec = O.LayerSpec(4096, 128, 1536, 8)
    g = geom(spec.hidden, spec.inter, spec.bits)
    slab = SlabStore(g, spec.experts, DEV)
    fill_slab_gpu(slab, range(spec.experts), seed=5)
    rng = np.random.default_rng(100 + n)
    gwb = O.bf16_round(rng.standard_normal((spec.experts, spec.hidden), dtype=np.float32)
                       * np.float32(0.02))
    xb = _x_bits(rng, n, spec.hidden)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", spec.experts, spec.top_k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV))
    ref_i, ref_w = O.softmax_topk(O.router_logits(xb, gwb), spec.top_k)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    used = sorted(set(ref_i.reshape(-1).tolist()))
    experts = {e: slot_to_expert(slab, e) for e in used}
    y = O.switch_glu_f64(xb, ref_i, experts)
    check_close(out.float().cpu().numpy(), O.combine_f64(y, ref_w), f"235B decode n={n}")


@pytest.mark.parametrize("n,scoring", [(1, "softmax"), (8, "softmax"), (8, "sigmoid")])
def test_decode_over_512_experts_vs_oracle(n, scoring):
    """1000 experts, D1024, I512, top-8, 4-bit.  Softmax takes the decode
    routing with 16 logits per lane (each block's routing prologue at n=1,
    the routing launch at n=8); sigmoid group scoring above 512 experts takes
    the general path (routing launch, dispatch, GEMVs).  Routing bit-exact,
    outputs within tolerance of the oracle."""
    K = _k()
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd._lib import geom
    e, ng, tg, scale = 1000, 8, 4, 2.5
    spec = O.LayerSpec(1024, e, 512, 8)
    g = geom(spec.hidden, spec.inter, spec.bits)
    slab = SlabStore(g, e, DEV)
    fill_slab_gpu(slab, range(e), seed=9)
    rng = np.random.default_rng(700 + n)
    gwb = O.bf16_round(rng.standard_normal((e, spec.hidden), dtype=np.float32)
                       * np.float32(0.02))
    bias = (rng.standard_normal(e, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    xb = _x_bits(rng, n, spec.hidden)
    table = torch.arange(e, dtype=torch.int32, device=DEV)
    logits = O.router_logits(xb, gwb)
    if scoring == "softmax":
        rc = K.route_cfg("softmax", e, spec.top_k)
        ref_i, ref_w = O.softmax_topk(logits, spec.top_k)
        kw = {}
    else:
        rc = K.route_cfg("sigmoid", e, spec.top_k, True, ng, tg, scale)
        ref_i, ref_w = O.sigmoid_group_topk(logits, bias, ng, tg, spec.top_k, True, scale)
        kw = {"score_bias": torch.from_numpy(bias).to(DEV)}
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV), **kw)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    used = sorted(set(ref_i.reshape(-1).tolist()))
    experts = {x: slot_to_expert(slab, x) for x in used}
    y = O.switch_glu_f64(xb, ref_i, experts)
    check_close(out.float().cpu().numpy(), O.combine_f64(y, ref_w), f"E1000 decode n={n}")
    slab.release()


def test_deepseek_shared_decode_vs_oracle():
    """Config 4 routing (sigmoid+bias, 8 groups/top-4, top-8, scale 2.5) + a
    shared expert, at reduced hidden size so the oracle stays fast."""
    K = _k()
    spec = O.LayerSpec(1024, 384, 512, 8, scoring="sigmoid", n_group=8, topk_group=4,
                       routed_scale=2.5, shared=1)
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd._lib import geom
    g = geom(spec.hidden, spec.inter, spec.bits)
    slab = SlabStore(g, spec.experts + 1, DEV)
    fill_slab_gpu(slab, range(spec.experts + 1), seed=9)
    rng = np.random.default_rng(9)
    gwb = O.bf16_round(rng.standard_normal((spec.experts, spec.hidden), dtype=np.float32)
                       * np.float32(0.02))
    bias = (rng.standard_normal(spec.experts, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    xb = _x_bits(rng, 2, spec.hidden)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("sigmoid", spec.experts, spec.top_k, True, 8, 4, 2.5)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV), score_bias=torch.from_numpy(bias).to(DEV),
                               shared_slot=spec.experts)
    ref_i, ref_w = O.sigmoid_group_topk(O.router_logits(xb, gwb), bias, 8, 4, 8, True, 2.5)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    used = sorted(set(ref_i.reshape(-1).tolist()))
    experts = {e: slot_to_expert(slab, e) for e in used}
    sh = slot_to_expert(slab, spec.experts)
    y = O.switch_glu_f64(xb, ref_i, experts)
    ref = O.combine_f64(y, ref_w, O.expert_ffn_f64(O.bf16_to_f32(xb), sh))
    check_close(out.float().cpu().numpy(), ref, "deepseek shared decode")


def test_qwen3_next_6bit_shared_gate_vs_oracle():
    """Config 5 shapes (D2048, E512, I512, top-10, 6-bit) + gated shared expert, N=8."""
    K = _k()
    spec = O.LayerSpec(2048, 512, 512, 10, bits=6, shared=1, shared_gate=True)
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd._lib import geom
    g = geom(spec.hidden, spec.inter, spec.bits)
    slab = SlabStore(g, spec.experts + 1, DEV)
    fill_slab_gpu(slab, range(spec.experts + 1), seed=11)
    rng = np.random.default_rng(11)
    gwb = O.bf16_round(rng.standard_normal((spec.experts, spec.hidden), dtype=np.float32)
                       * np.float32(0.02))
    sgb = O.bf16_round(rng.standard_normal((1, spec.hidden), dtype=np.float32) * np.float32(0.02))
    xb = _x_bits(rng, 8, spec.hidden)
    table = torch.arange(spec.experts, dtype=torch.int32, device=DEV)
    rc = K.route_cfg("softmax", spec.experts, spec.top_k)
    out, gi, gwt = K.moe_block(g, rc, slab.buf, table, bits_to_bf16_tensor(gwb, DEV),
                               bits_to_bf16_tensor(xb, DEV), shared_slot=spec.experts,
                               shared_gate=bits_to_bf16_tensor(sgb, DEV))
    ref_i, ref_w = O.softmax_topk(O.router_logits(xb, gwb), spec.top_k)
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    used = sorted(set(ref_i.reshape(-1).tolist()))
    experts = {e: slot_to_expert(slab, e) for e in used}
    sh = slot_to_expert(slab, spec.experts)
    x = O.bf16_to_f32(xb)
    gl = O.router_logits(xb, sgb)[:, 0].astype(np.float64)
    shared = O.expert_ffn_f64(x, sh) * (1.0 / (1.0 + np.exp(-gl)))[:, None]
    ref = O.combine_f64(O.switch_glu_f64(xb, ref_i, experts), ref_w, shared)
    check_close(out.float().cpu().numpy(), ref, "qwen3-next 6-bit shared gate")


def test_nonresident_expert_rows_are_zero():
    """A table entry of -1 yields exact zero rows (streaming.py:715-719)."""
    K = _k()
    spec = O.LayerSpec(1024, 8, 512, 2)
    gw, experts, _, _, _ = O.make_layer(spec, seed=3)
    g, slab = _slab_from_experts([experts[e] for e in range(8)], spec)
    table = torch.arange(8, dtype=torch.int32, device=DEV)
    table[3] = -1
    rng = np.random.default_rng(3)
    xb = _x_bits(rng, 4, spec.hidden)
    inds = np.array([[3, 1], [0, 3], [2, 5], [3, 7]], np.int32)
    y = K.switch_glu(g, slab.buf, table, 8, bits_to_bf16_tensor(xb, DEV),
                     torch.from_numpy(inds).to(DEV)).float().cpu().numpy()
    assert (y[inds == 3] == 0).all()
    ref = O.switch_glu_f64(xb, inds, experts)
    mask = inds != 3
    check_close(y[mask], ref[mask], "resident rows")
