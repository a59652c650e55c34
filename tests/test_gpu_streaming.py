"""GPU: the drop-in surface (StreamedSwitchGLU, MoE blocks, patch_model,
ExpertCache paging) and the committed golden fixtures through the HIP path.

The streamed seam must give the same bytes as the resident module for the
same experts (same kernels, the slot is the only difference), its residency
counters must follow the oracle's slot policy, and the blocks must match the
oracle's routing exactly and its float64 outputs within tests/util tolerance.
"""

from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from oracle import pmoe_oracle as O
from tests.util import bits_to_bf16_tensor, check_close, expert_to_comps, slot_to_expert

pytestmark = pytest.mark.gpu

DEV = "cuda"
G = Path(__file__).resolve().parent / "golden"


def _mods():
    from pagedmoe_amd import kernels, streaming
    return kernels, streaming


def _load(name):
    return np.load(G / name, allow_pickle=False)


# ---------------------------------------------------------------- golden fixtures

def test_golden_tiny_layer_on_gpu():
    K, S = _mods()
    f = _load("tiny_layer.npz")
    spec = O.LayerSpec(1024, 32, 512, 4)
    gw, experts, _, _, _ = O.make_layer(spec, seed=0)
    sw = S.QuantizedSwitchGLU(spec.hidden, spec.inter, spec.experts, spec.bits)
    for e in range(spec.experts):
        sw.load_expert(e, expert_to_comps(experts[e]))
    blk = S.SoftmaxMoEBlock(bits_to_bf16_tensor(f["gate_bits"], DEV), sw, spec.top_k)
    x = bits_to_bf16_tensor(f["x_bits"], DEV)
    out = blk(x)
    gi, gwt = blk.last_routing
    assert np.array_equal(gi.cpu().numpy(), f["inds"])
    assert np.array_equal(gwt.cpu().numpy(), f["weights"])
    check_close(out.float().cpu().numpy(), f["out"].astype(np.float64), "golden tiny layer out")
    logits = K.router_logits(x, bits_to_bf16_tensor(f["gate_bits"], DEV))
    assert np.array_equal(logits.cpu().numpy(), f["logits"])
    y = sw(x[:2], torch.from_numpy(f["inds"][:2]).to(DEV))
    check_close(y.float().cpu().numpy(), f["y"].astype(np.float64), "golden per-slot y")


def test_golden_routing_dispatch_quant_on_gpu():
    K, _ = _mods()
    f = _load("routing_sigmoid.npz")
    gi, gw = K.route_sigmoid_group_topk(torch.from_numpy(f["logits"]).to(DEV),
                                        torch.from_numpy(f["bias"]).to(DEV), 8, 4, 8, True, 2.5)
    assert np.array_equal(gi.cpu().numpy(), f["inds"])
    assert np.array_equal(gw.cpu().numpy(), f["weights"])
    f = _load("routing_softmax.npz")
    lg = torch.from_numpy(f["logits"]).to(DEV)
    for norm, ki, kw in ((True, "inds", "weights"), (False, "inds_nonorm", "weights_nonorm")):
        gi, gw = K.route_softmax_topk(lg, 10, norm)
        assert np.array_equal(gi.cpu().numpy(), f[ki])
        assert np.array_equal(gw.cpu().numpy(), f[kw])
    f = _load("dispatch.npz")
    d = K.dispatch(torch.from_numpy(f["ids"]).to(DEV), 128)
    for key in ("order", "counts", "offsets", "inv", "active"):
        assert np.array_equal(d[key].cpu().numpy(), f[key]), key
    f = _load("quant_format.npz")
    for bits in (4, 6):
        q, s, b = K.quantize(torch.from_numpy(f["w"]).to(DEV), bits)
        assert np.array_equal(q.cpu().numpy().view(np.uint32), f[f"q{bits}"])
        assert np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16), f[f"s{bits}"])
        assert np.array_equal(b.cpu().view(torch.int16).numpy().view(np.uint16), f[f"b{bits}"])
        deq = K.dequant(q, s, b, bits)
        assert np.array_equal(deq.cpu().view(torch.int16).numpy().view(np.uint16), f[f"deq{bits}"])


# ---------------------------------------------------------------- a toy model

class _Layer(nn.Module):
    def __init__(self, mlp):
        super().__init__()
        self.mlp = mlp


class _Model(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.layers = nn.ModuleList([_Layer(b) for b in blocks])


def _softmax_model(spec, n_layers, seed):
    """n_layers Qwen3-style blocks over resident QuantizedSwitchGLUs, oracle
    experts per layer (make_layer seeds seed+layer)."""
    _, S = _mods()
    blocks, oracle_layers = [], []
    for li in range(n_layers):
        gw, experts, _, sh, sg = O.make_layer(spec, seed=seed + li)
        sw = S.QuantizedSwitchGLU(spec.hidden, spec.inter, spec.experts, spec.bits,
                                  n_shared=spec.shared)
        for e in range(spec.experts):
            sw.load_expert(e, expert_to_comps(experts[e]))
        if spec.shared:
            sw.load_expert(spec.experts, expert_to_comps(sh[0]))
        sgt = None if sg is None else bits_to_bf16_tensor(sg, DEV)
        blocks.append(S.SoftmaxMoEBlock(bits_to_bf16_tensor(gw, DEV), sw, spec.top_k,
                                        shared_expert_gate=sgt))
        oracle_layers.append((gw, experts, sh, sg))
    return _Model(blocks), oracle_layers


def _resident_outputs(model, xs):
    with torch.no_grad():
        return [[layer.mlp.switch_mlp(x, i).clone() for x, i in step] for step, layer in
                zip([xs] * len(model.layers), model.layers)]


def test_find_switch_glus_order():
    _, S = _mods()
    spec = O.LayerSpec(1024, 8, 512, 2)
    model, _ = _softmax_model(spec, 3, seed=40)
    paths = [p for p, _ in S.find_switch_glus(model)]
    assert paths == [f"layers.{i}.mlp.switch_mlp" for i in range(3)]


def test_streamed_switch_paging_matches_resident_and_policy():
    """16 routed slots (reserve 4, budget 12) for 3 layers x 32 experts: the
    streamed seam pages experts in and out; every call's output equals the
    resident module's, and hits/misses/evictions equal the oracle policy's."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 3, seed=50)
    resident = [layer.mlp.switch_mlp for layer in model.layers]
    cache = S.build_cache_for(model, slots=16)
    streamed = S.patch_model(model, cache, predict_mode="off")
    assert not cache.stitched
    assert all(isinstance(layer.mlp.switch_mlp, S.StreamedSwitchGLU) for layer in model.layers)
    pol = O.SlotPolicy(16)
    rng = np.random.default_rng(51)
    for step in range(12):
        n = 1 + step % 3
        for li, (res, st) in enumerate(zip(resident, streamed)):
            x = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((n, spec.hidden),
                                                                     dtype=np.float32)), DEV)
            ids = np.stack([rng.choice(spec.experts, spec.top_k, replace=False) for _ in range(n)])
            ids = ids.astype(np.int32)
            ind = torch.from_numpy(ids).to(DEV)
            got = st(x, ind)
            ref = res(x, ind)
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (step, li)
            pol.step(st.layer_key, ids.reshape(-1))
            assert np.array_equal(cache.host_table(st.layer_key),
                                  pol.table(st.layer_key, spec.experts)), (step, li)
    s = cache.stats()
    assert (s["hits"], s["misses"], s["evictions"]) == (pol.hits, pol.misses, pol.evictions)
    assert s["evictions"] > 0 and s["hits"] > 0
    assert S.get_stats(model)["cache"]["misses"] == pol.misses
    cache.close()


def test_streamed_switch_stitched_when_all_fit():
    _, S = _mods()
    spec = O.LayerSpec(1024, 8, 512, 2)
    model, _ = _softmax_model(spec, 2, seed=60)
    resident = [layer.mlp.switch_mlp for layer in model.layers]
    cache = S.build_cache_for(model, slots=16)
    streamed = S.patch_model(model, cache)
    assert cache.stitched
    rng = np.random.default_rng(61)
    for res, st in zip(resident, streamed):
        assert np.array_equal(cache.host_table(st.layer_key),
                              np.arange(8, dtype=np.int32) + 8 * cache.layer_index(st.layer_key))
        x = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((5, spec.hidden),
                                                                 dtype=np.float32)), DEV)
        ind = torch.from_numpy(rng.integers(0, 8, (5, 2)).astype(np.int32)).to(DEV)
        assert torch.equal(st(x, ind).view(torch.int16), res(x, ind).view(torch.int16))
    assert cache.stats()["misses"] == 0
    cache.close()


@pytest.mark.parametrize("n", [1, 3])
def test_softmax_block_paged_vs_oracle(n):
    """Patched Qwen3-style model, experts paged through a 16-slot slab: each
    layer's routing is bit-exact and its output within tolerance of the
    float64 oracle."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, ol = _softmax_model(spec, 2, seed=70)
    cache = S.build_cache_for(model, slots=16)
    S.patch_model(model, cache)
    rng = np.random.default_rng(71 + n)
    for step in range(3):
        for li, layer in enumerate(model.layers):
            xb = O.bf16_round(rng.standard_normal((n, spec.hidden), dtype=np.float32))
            out = layer.mlp(bits_to_bf16_tensor(xb, DEV))
            gw, experts, _, _ = ol[li]
            ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts)
            gi, gwt = layer.mlp.last_routing
            assert np.array_equal(gi.cpu().numpy(), ref_i)
            assert np.array_equal(gwt.cpu().numpy(), ref_w)
            check_close(out.float().cpu().numpy(), ref, f"paged block step {step} layer {li}")
    assert cache.stats()["misses"] > 0
    cache.close()


def test_sigmoid_shared_block_paged_and_resident_vs_oracle():
    """DeepSeek-style routing with a shared expert: resident block (fused
    path) and paged block (route -> fetch -> experts) both match the oracle."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 64, 512, 6, scoring="sigmoid", n_group=8, topk_group=4,
                       routed_scale=2.5, shared=1)
    gw, experts, bias, sh, _ = O.make_layer(spec, seed=80)
    sw = S.QuantizedSwitchGLU(spec.hidden, spec.inter, spec.experts, spec.bits, n_shared=1)
    for e in range(spec.experts):
        sw.load_expert(e, expert_to_comps(experts[e]))
    sw.load_expert(spec.experts, expert_to_comps(sh[0]))
    blk = S.SigmoidGroupMoEBlock(bits_to_bf16_tensor(gw, DEV), torch.from_numpy(bias).to(DEV), sw,
                                 spec.top_k, spec.n_group, spec.topk_group, spec.routed_scale)
    model = _Model([blk])
    rng = np.random.default_rng(81)
    xb = O.bf16_round(rng.standard_normal((3, spec.hidden), dtype=np.float32))
    ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts, bias=bias, shared=sh)
    out_res = blk(bits_to_bf16_tensor(xb, DEV))
    gi, gwt = blk.last_routing
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out_res.float().cpu().numpy(), ref, "sigmoid shared resident")
    cache = S.build_cache_for(model, slots=20)
    S.patch_model(model, cache)
    assert not cache.stitched
    assert cache.shared_slot("layers.0.mlp.switch_mlp") == 20
    ex_sh = slot_to_expert(cache.slab, 20)
    assert np.array_equal(ex_sh.down.weight, sh[0].down.weight)
    out_pg = model.layers[0].mlp(bits_to_bf16_tensor(xb, DEV))
    gi, gwt = model.layers[0].mlp.last_routing
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    check_close(out_pg.float().cpu().numpy(), ref, "sigmoid shared paged")
    cache.close()


def test_streamed_switch_fetch_groups_match_resident():
    """8 routed slots, 8 tokens x top-4 over 32 experts: the layer's ids
    exceed the slab, so the seam runs several fetch groups; rows stay
    bit-identical to the resident module and nothing starves."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 2, seed=90)
    resident = [layer.mlp.switch_mlp for layer in model.layers]
    cache = S.build_cache_for(model, slots=8)
    streamed = S.patch_model(model, cache)
    rng = np.random.default_rng(91)
    for step in range(2):
        for res, st in zip(resident, streamed):
            x = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((8, spec.hidden),
                                                                     dtype=np.float32)), DEV)
            ids = np.stack([rng.choice(spec.experts, 4, replace=False) for _ in range(8)])
            ind = torch.from_numpy(ids.astype(np.int32)).to(DEV)
            assert torch.equal(st(x, ind).view(torch.int16), res(x, ind).view(torch.int16))
    s = cache.stats()
    assert s["group_passes"] >= 8 and s["slot_starved"] == 0
    cache.close()


def test_block_fetch_groups_with_gated_shared_vs_oracle():
    """Qwen3-Next-style block (softmax top-4 + sigmoid-gated shared expert)
    on an 8-slot slab: routed experts run in fetch groups, the shared expert
    from its own slot, and pmoe_combine merges them; routing bit-exact,
    output within tolerance of the float64 oracle."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4, shared=1, shared_gate=True)
    model, ol = _softmax_model(spec, 1, seed=95)
    cache = S.build_cache_for(model, slots=8)
    S.patch_model(model, cache)
    rng = np.random.default_rng(96)
    xb = O.bf16_round(rng.standard_normal((16, spec.hidden), dtype=np.float32))
    blk = model.layers[0].mlp
    out = blk(bits_to_bf16_tensor(xb, DEV))
    gw, experts, sh, sg = ol[0]
    ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts, shared=sh, shared_gate_bits=sg)
    gi, gwt = blk.last_routing
    assert np.array_equal(gi.cpu().numpy(), ref_i)
    assert np.array_equal(gwt.cpu().numpy(), ref_w)
    check_close(out.float().cpu().numpy(), ref, "grouped block + gated shared")
    assert cache.stats()["group_passes"] >= 2
    cache.close()


@pytest.mark.parametrize("shared,gate", [(False, False), (True, False), (True, True)])
def test_combine_entry_point_vs_oracle(shared, gate):
    K, _ = _mods()
    rng = np.random.default_rng(7 + shared + 2 * gate)
    n, k, d = 5, 6, 1024
    y = O.bf16_round(rng.standard_normal((n, k, d), dtype=np.float32))
    w = rng.random((n, k), dtype=np.float32)
    sy = O.bf16_round(rng.standard_normal((n, d), dtype=np.float32)) if shared else None
    sl = rng.standard_normal(n, dtype=np.float32) if gate else None
    got = K.combine(bits_to_bf16_tensor(y, DEV), torch.from_numpy(w).to(DEV),
                    None if sy is None else bits_to_bf16_tensor(sy, DEV),
                    None if sl is None else torch.from_numpy(sl).to(DEV))
    yf = O.bf16_to_f32(y)
    shf = None
    if shared:
        shf = O.bf16_to_f32(sy).astype(np.float64)
        if gate:
            shf = shf * (1.0 / (1.0 + np.exp(-sl.astype(np.float64))))[:, None]
    ref = O.combine_f64(yf.astype(np.float64), w, shf)
    check_close(got.float().cpu().numpy(), ref, "pmoe_combine")
    ref32 = O.combine_f32(yf, w, None if sy is None else O.bf16_to_f32(sy),
                          None if sl is None else O.psigmoid(sl))
    assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), ref32)


def test_paged_block_reads_experts_from_a_safetensors_checkpoint(tmp_path):
    """Experts paged from a quantized safetensors checkpoint
    (build_cache_for(model_path=...) -> HostExpertStore.from_checkpoint):
    the modules' own slabs are zeroed first, so every routed expert the
    layers use comes from the files; routing bit-exact and outputs within
    tolerance of the float64 oracle."""
    from safetensors.torch import save_file

    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, ol = _softmax_model(spec, 2, seed=90)
    tensors = {}
    for li, (_, experts, _, _) in enumerate(ol):
        for proj in ("gate", "up", "down"):
            qts = [getattr(experts[e], proj) for e in range(spec.experts)]
            pre = f"model.layers.{li}.mlp.switch_mlp.{proj}_proj"
            tensors[pre + ".weight"] = torch.from_numpy(
                np.stack([q.weight for q in qts]).astype(np.uint32).view(np.int32))
            for comp in ("scales", "biases"):
                a = np.stack([getattr(q, comp) for q in qts]).view(np.int16)
                tensors[f"{pre}.{comp}"] = torch.from_numpy(a).view(torch.bfloat16)
    save_file(tensors, str(tmp_path / "model.safetensors"))
    for _, m in S.find_switch_glus(model):
        m.slab.buf.zero_()
    cache = S.build_cache_for(model, slots=16, model_path=tmp_path)
    S.patch_model(model, cache)
    rng = np.random.default_rng(91)
    print("[checkpoint] paged block from safetensors", flush=True)
    for step in range(2):
        for li, layer in enumerate(model.layers):
            xb = O.bf16_round(rng.standard_normal((2, spec.hidden), dtype=np.float32))
            out = layer.mlp(bits_to_bf16_tensor(xb, DEV))
            gw, experts, _, _ = ol[li]
            ref_i, ref_w, _, ref = O.moe_layer_f64(spec, xb, gw, experts)
            gi, gwt = layer.mlp.last_routing
            assert np.array_equal(gi.cpu().numpy(), ref_i)
            assert np.array_equal(gwt.cpu().numpy(), ref_w)
            check_close(out.float().cpu().numpy(), ref, f"checkpoint paging step {step} layer {li}")
    assert cache.stats()["misses"] > 0
    cache.close()


# ---------------------------------------------------------------- prefill residency

def _replay_prefill(pol, layer, groups):
    """The oracle policy over one prefill call's fetch groups, in the order
    the seam issued them (a group opened while the previous one still held
    its slots, or after it gave them back)."""
    t, _, _ = pol.step_prefill(layer, groups[0])
    for how, ids in groups[1:]:
        if how == "after_done":
            pol.prefill_done(t)
            t, _, _ = pol.step_prefill(layer, ids)
        else:
            t2, _, _ = pol.step_prefill(layer, ids)
            pol.prefill_done(t)
            t = t2
    pol.prefill_done(t)


@pytest.mark.parametrize("stage", [6, 64])
def test_prefill_groups_keep_the_decode_hot_set(stage, monkeypatch):
    """32-token calls take the prefill policy (cache.py:2347-2453 with
    prefill=True): hits are not touched, misses never evict, and groups whose
    copies run under the previous group's compute give rows bit-identical to
    the resident module.  With a 6-slot stage a call needs several groups
    that reuse stage slots; with 64, one group.  Tables and counters follow
    the oracle policy replayed over the same groups, and the decode hot set
    survives the prefill.  Prefill-ahead is off here: the replay covers the
    group policy only (a claimed prefill-ahead read counts as a hit, where
    the replay sees a miss); its own tests are the PREFILL_AHEAD trace and
    test_prefill_ahead_keeps_outputs_and_claims_reads."""
    from pagedmoe_amd import config
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore

    monkeypatch.setattr(config, "PREFILL_AHEAD", False)
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 2, seed=120)
    resident = [layer.mlp.switch_mlp for layer in model.layers]
    glus = S.find_switch_glus(model)
    g = glus[0][1].geom
    store = HostExpertStore(g, 2, spec.experts)
    for li, (_, m) in enumerate(glus):
        for e in range(spec.experts):
            store.write_from_slot(li, e, m.slab, e)
    cache = ExpertCache(g, 16, [p for p, _ in glus], spec.experts, host_store=store,
                        stage_slots=stage)
    streamed = S.patch_model(model, cache, predict_mode="off")
    assert not cache.stitched
    pol = O.SlotPolicy(16)
    pol.set_stage(cache.stage_first, stage)
    rng = np.random.default_rng(121)
    hot = [3, 7, 11, 19]

    def call(li, n, ids):
        x = bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((n, spec.hidden),
                                                                 dtype=np.float32)), DEV)
        ind = torch.from_numpy(ids.astype(np.int32)).to(DEV)
        got = streamed[li](x, ind)
        ref = resident[li](x, ind)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (li, n)

    for _ in range(3):  # decode: the hot set becomes resident with reuse credit
        for li in range(2):
            ids = np.array([hot], dtype=np.int32)
            call(li, 1, ids)
            pol.step(streamed[li].layer_key, ids.reshape(-1))
    ev0 = cache.stats()["evictions"]
    for li in range(2):
        ids = np.stack([rng.choice(spec.experts, spec.top_k, replace=False) for _ in range(32)])
        call(li, 32, ids)
        groups = streamed[li].last_groups
        _replay_prefill(pol, streamed[li].layer_key, groups)
        if stage == 6:
            assert len(groups) >= 3, groups
        for lk in (s.layer_key for s in streamed):
            assert np.array_equal(cache.host_table(lk), pol.table(lk, spec.experts)), lk
    st = cache.stats()
    assert st["evictions"] == ev0, "a prefill call evicted"
    assert (st["hits"], st["misses"]) == (pol.hits, pol.misses)
    for s in streamed:
        t = cache.host_table(s.layer_key)
        assert all(t[e] >= 0 for e in hot), "the decode hot set was flushed by a prefill"
    # the device rows are the persistent tables again (the groups' held
    # slots are not visible once the call is over)
    for s in streamed:
        assert not cache.table_dirty(s.layer_key)
        assert np.array_equal(cache.device_table(s.layer_key), cache.host_table(s.layer_key))
    cache.close()
    store.close()


def test_flow_table_republishes_rows_another_layer_evicted():
    """Layer 0's fetch evicts layer 1's expert; layer 1's device row is then
    stale until flow_table(layer 1) republishes it (cache.py:821-859), after
    which it shows -1 for that expert."""
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore

    _, S = _mods()
    spec = O.LayerSpec(1024, 16, 512, 4)
    model, _ = _softmax_model(spec, 2, seed=130)
    glus = S.find_switch_glus(model)
    g = glus[0][1].geom
    store = HostExpertStore(g, 2, spec.experts)
    for li, (_, m) in enumerate(glus):
        for e in range(spec.experts):
            store.write_from_slot(li, e, m.slab, e)
    keys = [p for p, _ in glus]
    cache = ExpertCache(g, 8, keys, spec.experts, host_store=store, stage_slots=0)  # budget 4

    device_row = cache.device_table
    cache.fetch(keys[1], [5])
    cache.fetch(keys[0], [0, 1, 2])
    torch.cuda.synchronize()
    assert device_row(keys[1])[5] >= 0
    assert not cache.table_dirty(keys[1])
    cache.fetch(keys[0], [3])            # 5 resident > budget 4: layer 1's 5 is the LRU head
    assert cache.host_table(keys[1])[5] == -1
    assert cache.table_dirty(keys[1])
    assert device_row(keys[1])[5] >= 0   # stale until republished
    cache.flow_table(keys[1])
    assert device_row(keys[1])[5] == -1
    assert not cache.table_dirty(keys[1])
    cache.close()
    store.close()


def test_fused_prefill_streams_the_experts_once_per_prompt(monkeypatch):
    """Fused prefill pass (prefill_fused.py) on a 2-layer toy decoder whose
    MoE blocks page experts through a 16-slot cache (fetch groups overlapping
    the previous group's compute): a 96-token call with 32-row attention
    splits runs each MoE block once over all 96 tokens; chunking the model
    call instead runs each MoE three times.

    The fused and the stock call run attention as different GEMM shapes
    (3 x 32 rows against 96 rows), so their MoE inputs may differ in the
    last bits, and a token whose k-th and (k+1)-th router logits nearly tie
    may then route differently -- a legitimate difference, not a paging
    error.  So every MoE call of both runs is checked on its own input:
    routing bit-exact and outputs within tolerance of the float64 oracle.
    Attention equivalence is checked separately (MoE inputs close), and the
    tokens whose routing differs between the runs are reported with their
    logit margins."""
    import math

    from pagedmoe_amd import config, prefill_fused as PF

    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)

    class Cache:
        def __init__(self):
            self.k = self.v = None

        @property
        def offset(self):
            return 0 if self.k is None else self.k.shape[2]

        def update_and_fetch(self, k, v):
            self.k = k if self.k is None else torch.cat([self.k, k], 2)
            self.v = v if self.v is None else torch.cat([self.v, v], 2)
            return self.k, self.v

    class Attn(nn.Module):
        n_heads = 4

        def __init__(self, seed):
            super().__init__()
            g = torch.Generator(device=DEV).manual_seed(seed)
            self.w = [torch.randn(1024, 1024, generator=g, device=DEV) / 32 for _ in range(4)]

        def forward(self, x, mask, cache):
            b, t, d = x.shape
            q, k, v = (z.reshape(b, t, 4, d // 4).transpose(1, 2).contiguous()
                       for z in (x @ self.w[0], x @ self.w[1], x @ self.w[2]))
            k, v = cache.update_and_fetch(k, v)
            s = q @ k.transpose(-1, -2).contiguous() / math.sqrt(d // 4) + mask
            return (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(b, t, d) @ self.w[3]

    class Norm(nn.Module):
        def forward(self, x):
            return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    class Layer(nn.Module):
        def __init__(self, moe, seed):
            super().__init__()
            self.self_attn, self.mlp = Attn(seed), moe
            self.input_layernorm, self.post_attention_layernorm = Norm(), Norm()

        def forward(self, x, mask=None, cache=None):
            h = x + self.self_attn(self.input_layernorm(x), mask, cache)
            return h + self.mlp(self.post_attention_layernorm(h)).float()

    moe_model, oracle_layers = _softmax_model(spec, 2, seed=140)
    cache = S.build_cache_for(moe_model, slots=16)
    S.patch_model(moe_model, cache)
    model = nn.Module()
    model.layers = nn.ModuleList([Layer(moe_model.layers[i].mlp, 141 + i) for i in range(2)])

    def run(x, caches):
        t, off = x.shape[1], caches[0].offset
        q = torch.arange(off, off + t, device=DEV)[:, None]
        mask = torch.where(torch.arange(off + t, device=DEV)[None, :] <= q, 0.0, float("-inf"))
        for layer, c in zip(model.layers, caches):
            x = layer(x, mask, c)
        return x

    calls = []                              # (layer, bf16 input, output, inds, weights)
    for li, layer in enumerate(model.layers):
        orig = type(layer.mlp).forward

        def rec(x, m=layer.mlp, o=orig, li=li):
            y = o(m, x)
            inds, w = m.last_routing
            calls.append((li, x.to(torch.bfloat16).reshape(-1, spec.hidden).clone(), y.clone(),
                          inds.clone(), w.clone()))
            return y
        layer.mlp.forward = rec

    gen = torch.Generator(device=DEV).manual_seed(142)
    x = torch.randn(1, 96, 1024, device=DEV, generator=gen)
    with torch.no_grad():
        ref = run(x, [Cache(), Cache()])
        stock_calls = list(calls)
        monkeypatch.setattr(config, "ATTN_SUB_CHUNK", 32)
        assert PF.install(model)
        try:
            calls.clear()
            got = run(x, [Cache(), Cache()])
            fused_calls = list(calls)
            # one MoE pass per layer for the whole prompt, three attention splits
            assert [c[1].shape[0] for c in fused_calls] == [96, 96]
            assert [c[1].shape[0] for c in stock_calls] == [96, 96]
            assert all(PF.row_splits(layer, 96, 0) == [(0, 32), (32, 64), (64, 96)]
                       for layer in model.layers)
            calls.clear()
            caches = [Cache(), Cache()]
            for c0 in range(0, 96, 32):     # the model call chunked instead
                run(x[:, c0:c0 + 32], caches)
            assert [c[1].shape[0] for c in calls] == [32, 32] * 3
        finally:
            PF.uninstall()
    torch.cuda.synchronize()

    # every MoE call against the oracle on its own input
    for tag, recs in (("stock", stock_calls), ("fused", fused_calls)):
        for li, xb, y, inds, w in recs:
            gw, experts, _, _ = oracle_layers[li]
            xb_bits = xb.view(torch.int16).cpu().numpy().view(np.uint16)
            ref_i, ref_w, _, ref_out = O.moe_layer_f64(spec, xb_bits, gw, experts)
            assert np.array_equal(inds.cpu().numpy(), ref_i), (tag, li)
            assert np.array_equal(w.cpu().numpy(), ref_w), (tag, li)
            check_close(y.float().reshape(-1, spec.hidden).cpu().numpy(), ref_out,
                        f"{tag} prefill layer {li} MoE vs oracle")

    # attention equivalence, and the routing differences it may cause
    for (li, xs, _, i_s, _), (_, xf, _, i_f, _) in zip(stock_calls, fused_calls):
        a, b = xs.float(), xf.float()
        rel = ((a - b).norm() / a.norm()).item()
        assert rel < 1e-2, (li, rel)
        logits = O.router_logits(xs.view(torch.int16).cpu().numpy().view(np.uint16),
                                 oracle_layers[li][0])
        srt = -np.sort(-logits, axis=-1)
        margin = srt[:, spec.top_k - 1] - srt[:, spec.top_k]
        flipped = np.nonzero((np.sort(i_s.cpu().numpy(), -1) !=
                              np.sort(i_f.cpu().numpy(), -1)).any(-1))[0]
        print(f"[fused prefill] layer {li}: MoE input rel diff {rel:.2e}, "
              f"{int((a != b).any(-1).sum())} of 96 rows differ in some bf16 element, "
              f"routing differs on tokens {flipped.tolist()} "
              f"(their top-{spec.top_k} margins {margin[flipped].tolist()}); "
              f"smallest margin {margin.min():.3e}", flush=True)
    out_rel = ((got - ref).norm() / ref.norm()).item()
    print(f"[fused prefill] model output rel L2 diff fused vs stock {out_rel:.2e}", flush=True)
    cache.close()


# ---------------------------------------------------------------- flow decode

def _flow_model(monkeypatch, seed, slots=16):
    from pagedmoe_amd import config
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, ol = _softmax_model(spec, 2, seed=seed)
    cache = S.build_cache_for(model, slots=slots)
    ring = S.patch_model(model, cache)
    monkeypatch.setattr(config, "FLOW_WARMUP", 1)
    monkeypatch.setattr(config, "FLOW_WARM_HIT", 0.0)
    monkeypatch.setattr(config, "FLOW_MAX_CRIT", 0.0)     # these tests want flow to stay on
    ring.flow = True
    return spec, model, ol, cache, ring


def _masked_ref(spec, xb, layer_oracle, table):
    gw, experts, _, _ = layer_oracle
    ref_i, ref_w, y, _ = O.moe_layer_f64(spec, xb, gw, experts)
    keep = (table[ref_i] >= 0).astype(np.float64)        # non-resident: zero row
    return ref_i, ref_w, O.combine_f64(y * keep[..., None], ref_w), keep


def test_flow_decode_tokens_without_host_sync(monkeypatch):
    """Flow decode (streaming.py:675-724, cache.py:861-910): after one
    per-layer warm-up token, each token's layers run with no host round trip
    (the routed-id sync is never reached), against the device table
    published at the token's start.  Every flow token's routing is bit-exact
    and its output equals the oracle with the non-resident experts' rows
    zeroed; the last token's misses are admitted at the next token's start,
    so a repeated routing's experts become resident a few tokens later."""
    _, S = _mods()
    spec, model, ol, cache, ring = _flow_model(monkeypatch, seed=150)
    assert not cache.stitched
    rng = np.random.default_rng(151)
    xs = [O.bf16_round(rng.standard_normal((1, spec.hidden), dtype=np.float32))
          for _ in range(2)]
    orig = S.StreamedSwitchGLU.routed_ids
    in_flow = {"on": False}

    def guarded(self, indices):
        assert not in_flow["on"], "a flow token synced on its routed ids"
        return orig(self, indices)

    monkeypatch.setattr(S.StreamedSwitchGLU, "routed_ids", guarded)
    kept = []
    for t in range(12):
        xb = xs[min(t, 1)]                  # warm-up token on x0, then x1 repeated: its
        # experts miss at first, are admitted, and become resident
        in_flow["on"] = t >= 1
        outs = [layer.mlp(bits_to_bf16_tensor(xb, DEV)) for layer in model.layers]
        torch.cuda.synchronize()
        assert ring.token_flow == (t >= 1)
        if t == 0:
            continue
        for li, layer in enumerate(model.layers):
            lk = ring[li].layer_key
            table = cache.host_table(lk)
            assert np.array_equal(cache.device_table(lk), table), (t, li)
            ref_i, ref_w, ref, keep = _masked_ref(spec, xb, ol[li], table)
            gi, gwt = layer.mlp.last_routing
            assert np.array_equal(gi.cpu().numpy(), ref_i) and np.array_equal(gwt.cpu().numpy(), ref_w)
            check_close(outs[li].float().cpu().numpy(), ref, f"flow token {t} layer {li}")
            kept.append(keep.mean())
    assert ring.flow_tokens == 11 and ring.sync_tokens == 1
    assert kept[-1] == 1.0 and min(kept) < 1.0    # misses got admitted
    assert cache.stats()["flow_admits"] > 0
    cache.close()


def test_flow_token_captured_in_a_graph(monkeypatch):
    """A flow token's two MoE layers captured once as a HIP graph and
    replayed after each begin_token (auto_pump off): residency changes between
    replays reach the graph through the republished device tables, and every
    replay matches the oracle with the non-resident rows zeroed."""
    spec, model, ol, cache, ring = _flow_model(monkeypatch, seed=160)
    rng = np.random.default_rng(161)
    x = torch.empty((1, spec.hidden), dtype=torch.bfloat16, device=DEV)
    outs = [torch.empty((1, spec.hidden), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    xs = [O.bf16_round(rng.standard_normal((1, spec.hidden), dtype=np.float32))
          for _ in range(2)]
    x.copy_(bits_to_bf16_tensor(xs[0], DEV))
    for _ in range(2):                      # warm-up token, then one eager flow token
        for layer in model.layers:
            layer.mlp(x)
    torch.cuda.synchronize()
    assert ring.token_flow
    ring.auto_pump = False
    ring.begin_token()

    def token():
        for li, layer in enumerate(model.layers):
            outs[li].copy_(layer.mlp(x))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        token()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    ring.begin_token()
    with torch.cuda.graph(graph):
        token()
    torch.cuda.synchronize()
    for rep in range(6):
        xb = xs[rep % 2]
        x.copy_(bits_to_bf16_tensor(xb, DEV))
        ring.begin_token(replayed=rep > 0)
        tables = [cache.host_table(ring[li].layer_key) for li in range(2)]
        print(f"[flow] graph replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for li in range(2):
            _, _, ref, _ = _masked_ref(spec, xb, ol[li], tables[li])
            check_close(outs[li].float().cpu().numpy(), ref, f"flow graph replay {rep} layer {li}")
    ring.auto_pump = True
    cache.close()


# ---------------------------------------------------------------- speculative prefetch

def test_route_prediction_speculates_without_changing_outputs():
    """4 layers x 32 experts, 24 routed slots: after each decode layer the
    routers of the layers two and three ahead run on its hidden state, their
    guesses are read into free slots behind the layer's compute, and the
    target layer's fetch claims the ones it routes (cache.py:2853,
    streaming.py:2013-2299).  Outputs stay bit-identical to a
    paged twin with prediction off; every fetch and speculate call, replayed
    on the oracle policy
    (copies settled in between), gives the same tables and counters; the
    residual-stream inputs (each layer adds a small update) make the guesses
    useful, and precision is counted."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 4, seed=170)
    twin, _ = _softmax_model(spec, 4, seed=170)        # same weights, prediction off
    cache = S.build_cache_for(model, slots=24)
    ring = S.patch_model(model, cache, predict_mode="on")
    twin_cache = S.build_cache_for(twin, slots=24)
    S.patch_model(twin, twin_cache, predict_mode="off")
    assert ring.predict_depth == 3 and all(s.pred is not None for s in ring)
    cache.spec_log = []
    rng = np.random.default_rng(171)
    for t in range(10):
        h = torch.from_numpy(rng.standard_normal((1, spec.hidden), dtype=np.float32)).to(DEV)
        for li, layer in enumerate(model.layers):
            xb = h.to(torch.bfloat16)
            got = layer.mlp(xb)
            ref = twin.layers[li].mlp(xb)
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (t, li)
            torch.cuda.synchronize()
            cache.sync_spec()
            h = h + 0.05 * torch.from_numpy(rng.standard_normal(
                (1, spec.hidden), dtype=np.float32)).to(DEV)
    pol = O.SlotPolicy(24)
    keys = [s.layer_key for s in ring]
    for op in cache.spec_log:
        if op[0] == "fetch":
            pol.settle()
            pol.step(op[1], op[2])
        else:
            pol.speculate(op[1], op[2], op[3])
    for lk in keys:
        assert np.array_equal(cache.host_table(lk), pol.table(lk, spec.experts)), lk
    st = cache.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (pol.hits, pol.misses, pol.evictions)
    r = ring.stats()
    assert st["spec_started"] > 0 and st["spec_claims"] > 0 and st["spec_claims_late"] == 0
    assert r["pred_issued"] > 0 and r["pred_precision"] > 0.3, r
    print(f"[spec] {r} {st['spec_started']} started, {st['spec_claims']} claimed", flush=True)
    assert st["misses"] < twin_cache.stats()["misses"]     # claimed guesses were misses there
    cache.close()
    twin_cache.close()


# ---------------------------------------------------------------- slot-safety ledger

def test_speculation_overlapping_compute_is_bit_identical_and_race_free():
    """Route prediction with nothing waited for between layers (no device
    synchronise, no wait for the guesses): guesses read into free slots
    while later layers compute, and are claimed by their targets.  Outputs
    stay bit-identical to a prediction-off twin, and the native slot ledger
    (copy engines + slab + computes) replayed by verify.SlotLedger shows no
    write racing a read."""
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 4, seed=170)
    twin, _ = _softmax_model(spec, 4, seed=170)
    cache = S.build_cache_for(model, slots=24)
    ring = S.patch_model(model, cache, predict_mode="on")
    twin_cache = S.build_cache_for(twin, slots=24)
    S.patch_model(twin, twin_cache, predict_mode="off")
    led = cache.verify_slots(True)
    rng = np.random.default_rng(172)
    outs, refs = [], []
    for t in range(12):
        h = torch.from_numpy(rng.standard_normal((1, spec.hidden), dtype=np.float32)).to(DEV)
        for li, layer in enumerate(model.layers):
            xb = h.to(torch.bfloat16)
            outs.append(layer.mlp(xb))
            refs.append(twin.layers[li].mlp(xb))
            h = h + 0.05 * torch.from_numpy(rng.standard_normal(
                (1, spec.hidden), dtype=np.float32)).to(DEV)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(outs, refs)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), i
    st = cache.stats()
    print(f"[ledger spec] {led.report()} started {st['spec_started']} claims "
          f"{st['spec_claims']} late {st['spec_claims_late']}", flush=True)
    assert st["spec_started"] > 0 and st["spec_claims"] > 0
    assert led.counts["BATCH_JOIN"] > 0 and led.counts["COMPUTE"] == 48
    assert led.conflicts == [], led.conflicts[:3]
    assert st["slab_conflicts"] == 0
    cache.close()
    twin_cache.close()


def test_prefill_groups_and_flow_under_the_slot_ledger(monkeypatch):
    """The native event stream of prefill fetch groups (copies under the
    previous group's compute, stage slots) and of flow decode (admit behind
    a fence, install once landed, rows republished) replayed through the
    slot ledger: no conflicts, and the prefill outputs match the oracle."""
    from pagedmoe_amd import config

    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, ol = _softmax_model(spec, 2, seed=180)
    cache = S.build_cache_for(model, slots=16, stage_slots=4)   # 20 slots a group: several
    ring = S.patch_model(model, cache)
    led = cache.verify_slots(True)
    rng = np.random.default_rng(181)
    xb = O.bf16_round(rng.standard_normal((96, spec.hidden), dtype=np.float32))
    for li, layer in enumerate(model.layers):
        out = layer.mlp(bits_to_bf16_tensor(xb, DEV))
        torch.cuda.synchronize()
        gw, experts, _, _ = ol[li]
        _, _, _, ref = O.moe_layer_f64(spec, xb, gw, experts)
        check_close(out.float().cpu().numpy(), ref, f"ledger prefill layer {li}")
    groups = [len(s.last_groups) for s in ring]
    monkeypatch.setattr(config, "FLOW_WARMUP", 1)
    monkeypatch.setattr(config, "FLOW_WARM_HIT", 0.0)
    monkeypatch.setattr(config, "FLOW_MAX_CRIT", 0.0)
    ring.flow = True
    for t in range(10):
        xt = O.bf16_round(rng.standard_normal((1, spec.hidden), dtype=np.float32))
        for layer in model.layers:
            layer.mlp(bits_to_bf16_tensor(xt, DEV))
    torch.cuda.synchronize()
    print(f"[ledger prefill+flow] groups per layer {groups}, {led.report()}, "
          f"flow tokens {ring.flow_tokens}", flush=True)
    assert max(groups) >= 2 and ring.flow_tokens >= 8
    assert led.counts["ISSUE"] > 0 and led.counts["BATCH_JOIN"] > 0
    assert led.conflicts == [], led.conflicts[:3]
    cache.close()


# ---------------------------------------------------------------- closed stitch

class _TrimKV:
    """KV cache with mlx-lm's interface: offset, update_and_fetch, trim(n)."""

    def __init__(self):
        self.k = self.v = None

    @property
    def offset(self):
        return 0 if self.k is None else self.k.shape[2]

    def update_and_fetch(self, k, v):
        self.k = k if self.k is None else torch.cat([self.k, k], 2)
        self.v = v if self.v is None else torch.cat([self.v, v], 2)
        return self.k, self.v

    def trim(self, n):
        n = min(n, self.offset)
        self.k, self.v = self.k[:, :, :self.offset - n], self.v[:, :, :self.offset - n]
        return n


def _closed_decoder(spec, seed, slots):
    """A 2-layer pre-norm decoder (attention with a trimmable KV cache, MoE
    blocks paged through ``slots`` routed slots) and its ring."""
    import math

    _, S = _mods()
    moe_model, ol = _softmax_model(spec, 2, seed=seed)
    cache = S.build_cache_for(moe_model, slots=slots)
    ring = S.patch_model(moe_model, cache, predict_mode="off")

    class Attn(nn.Module):
        def __init__(self, s):
            super().__init__()
            g = torch.Generator(device=DEV).manual_seed(s)
            self.w = [torch.randn(spec.hidden, spec.hidden, generator=g, device=DEV)
                      / spec.hidden ** 0.5 for _ in range(4)]

        def forward(self, x, cache):
            b, t, d = x.shape
            q, k, v = (z.reshape(b, t, 4, d // 4).transpose(1, 2).contiguous()
                       for z in (x @ self.w[0], x @ self.w[1], x @ self.w[2]))
            k, v = cache.update_and_fetch(k, v)
            s = q @ k.transpose(-1, -2).contiguous() / math.sqrt(d // 4)
            o = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(b, t, d)
            return 0.05 * (o @ self.w[3])          # small: the residual keeps routing steady

    class Decoder(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = nn.ModuleList([Attn(seed + 10 + i) for i in range(2)])
            self.moe = nn.ModuleList([moe_model.layers[i].mlp for i in range(2)])

        def forward(self, x, cache=None):
            for a, m, c in zip(self.attn, self.moe, cache):
                x = x + a(x, c)
                x = x + m(x).float()
            return x

    dec = Decoder()
    dec._pagedmoe_ring, dec._pagedmoe_cache = ring, cache
    return dec, cache, ring, ol


def test_closed_stitch_keeps_exact_tokens_and_replays_misses(monkeypatch):
    """Closed stitch (streaming.py:2691-2870): after warm per-layer tokens
    the decode token runs both MoE layers against the live tables with no
    routed-id sync; its device miss count decides.  Every token -- kept or
    replayed after a forced miss -- is bit-identical to a per-layer twin,
    and the KV caches end in the same state."""
    from pagedmoe_amd import closed as C, config

    _, S = _mods()
    monkeypatch.setattr(config, "STITCH_PARTIAL", True)
    spec = O.LayerSpec(1024, 32, 512, 4)
    dec, cache, ring, _ = _closed_decoder(spec, 190, slots=24)
    ref, ref_cache, _, _ = _closed_decoder(spec, 190, slots=24)
    assert not cache.stitched and C.install(dec)
    rng = np.random.default_rng(191)
    hot = [torch.from_numpy(rng.standard_normal((1, 1, spec.hidden), dtype=np.float32)).to(DEV)
           for _ in range(2)]
    cold = [torch.from_numpy(rng.standard_normal((1, 1, spec.hidden), dtype=np.float32)).to(DEV)
            for _ in range(3)]
    kv, kv_ref = [_TrimKV(), _TrimKV()], [_TrimKV(), _TrimKV()]
    syncs = {"n": 0}
    orig = S.StreamedSwitchGLU.routed_ids

    def counted(self, indices):
        if self.cache is cache:            # the closed-stitch model's layers only
            syncs["n"] += 1
        return orig(self, indices)

    monkeypatch.setattr(S.StreamedSwitchGLU, "routed_ids", counted)
    seq = [hot[t % 2] for t in range(12)] + [cold[0]] + [hot[t % 2] for t in range(4)]
    seq += [cold[1], cold[2]]
    log = []
    for t, x in enumerate(seq):
        ok, rep, n0 = ring.closed_ok, ring.closed_replay, syncs["n"]
        with torch.no_grad():
            y = dec(x, cache=kv)
            y_ref = ref(x, cache=kv_ref)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"token {t}: closed-stitch output differs from per-layer"
        kind = ("kept" if ring.closed_ok > ok else "replayed" if ring.closed_replay > rep
                else "per-layer")
        if kind == "kept":
            assert syncs["n"] == n0, f"token {t}: a kept closed token synced per layer"
        log.append(kind)
    print(f"[closed] {log} ok={ring.closed_ok} replay={ring.closed_replay}", flush=True)
    assert ring.closed_ok >= 3 and ring.closed_replay >= 1
    assert "replayed" in log[12:13] or "replayed" in log[17:]
    for a, b in zip(kv, kv_ref):
        assert a.offset == b.offset == len(seq)
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    assert get_stats_ring(dec)["closed_ok"] == ring.closed_ok
    cache.close()
    ref_cache.close()


def get_stats_ring(model):
    _, S = _mods()
    return S.get_stats(model)["ring"]


# ---------------------------------------------------------------- prefill-time prediction

def test_native_prefill_ahead_known_answer():
    """The native policy on the hand-worked PREFILL_AHEAD trace
    (tests/slot_kats.py, from cache.py:2580-2650), with real reads: guesses
    take free slots above the floor then stage slots above its floor; the
    next layer's prefill group claims four of them (no read), misses two,
    hands back the rest; the claimed slots hold the host store's bytes."""
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore
    from tests import slot_kats

    kat = slot_kats.PREFILL_AHEAD
    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)
    model, _ = _softmax_model(spec, 2, seed=200)
    glus = S.find_switch_glus(model)
    g = glus[0][1].geom
    store = HostExpertStore(g, 2, spec.experts)
    for li, (_, m) in enumerate(glus):
        for e in range(spec.experts):
            store.write_from_slot(li, e, m.slab, e)
    keys = [p for p, _ in glus]
    cache = ExpertCache(g, kat["slots"], keys, spec.experts, host_store=store,
                        stage_slots=kat["stage"][1])
    assert cache.stage_first == kat["stage"][0]
    led = cache.verify_slots(True)
    cache.fetch(keys[0], kat["warm"])
    cache.spec_fence()
    n = cache.prefill_ahead(keys[1], kat["ahead"], kat["free_floor"], kat["stage_floor"])
    assert n == len(kat["started"])
    grp = cache.fetch_prefill(keys[1], kat["prefill"])
    assert grp.n_miss == len(kat["prefill_placed"]) and grp.n_unplaced == 0
    cache.publish_group(grp)
    cache.join()
    cache.note_compute(keys[1])
    row = cache.device_table(keys[1])
    assert {e: int(row[e]) for e in kat["prefill"]} == kat["compute_row"]
    for e, slot in kat["compute_row"].items():
        assert np.array_equal(cache.slab.slot_bytes(slot).cpu().numpy(),
                              store.expert_view(1, e)), (e, slot)
    cache.sync_spec()
    cache.drop_staged()
    cache.prefill_done(grp)
    t1 = cache.host_table(keys[1])
    assert {e: int(s) for e, s in enumerate(t1) if s >= 0} == kat["after"]
    st = cache.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (kat["hits"], kat["misses"],
                                                           kat["evictions"])
    assert st["prefill_ahead_reads"] == 7 and st["prefill_ahead_used"] == 4
    assert cache.capacity()[:2] == (len(kat["free_after"]), len(kat["stage_after"]))
    assert led.conflicts == [], led.conflicts[:3]
    cache.close()
    store.close()


def test_prefill_ahead_keeps_outputs_and_claims_reads(monkeypatch):
    """A 4-layer, 96-token prefill through a 20-slot cache (48 stage slots) on a residual
    stream: with prefill-time prediction each layer starts the next one's
    predicted reads after its own; the next layer claims the ones it routes.
    Outputs are bit-identical to a prediction-off twin, the native ledger
    shows no race, and fewer demand reads wait at the layer boundaries."""
    from pagedmoe_amd import config

    _, S = _mods()
    spec = O.LayerSpec(1024, 32, 512, 4)

    def build(ahead):
        model, _ = _softmax_model(spec, 4, seed=210)
        cache = S.build_cache_for(model, slots=20, stage_slots=48)
        S.patch_model(model, cache, predict_mode="off")
        return model, cache

    model, cache = build(True)
    twin, twin_cache = build(False)
    led = cache.verify_slots(True)
    rng = np.random.default_rng(211)
    h0 = rng.standard_normal((96, spec.hidden), dtype=np.float32)
    steps = [0.05 * rng.standard_normal((96, spec.hidden), dtype=np.float32) for _ in range(4)]
    for m, on in ((model, True), (twin, False)):
        monkeypatch.setattr(config, "PREFILL_AHEAD", on)
        h = torch.from_numpy(h0).to(DEV)
        outs = []
        for li, layer in enumerate(m.layers):
            outs.append(layer.mlp(h.to(torch.bfloat16)))
            h = h + torch.from_numpy(steps[li]).to(DEV)
        torch.cuda.synchronize()
        if on:
            got = outs
        else:
            ref = outs
    for li, (a, b) in enumerate(zip(got, ref)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), li
    st, st_ref = cache.stats(), twin_cache.stats()
    print(f"[prefill ahead] reads {st['prefill_ahead_reads']} used {st['prefill_ahead_used']} "
          f"skipped {st['prefill_ahead_skipped']}; demand misses {st['misses']} vs "
          f"{st_ref['misses']} without; ledger {led.report()}", flush=True)
    assert st["prefill_ahead_reads"] > 0 and st["prefill_ahead_used"] > 0
    assert st["misses"] < st_ref["misses"]
    assert led.conflicts == [], led.conflicts[:3]
    cache.close()
    twin_cache.close()
