"""GPU: the DeepSeek-V3/Kimi-K2-shaped paged decode at its full shape.

hidden 7168, 384 routed experts + 1 shared, moe_intermediate 2048, 4-bit
g64; a 96-slot HBM slab over a pinned host store of all 384 experts
(9.5 GB); batch 1.  Expert ids follow the seeded Zipf(1.1) trace of
tests/golden/make_golden.py.  Checked against the oracle:

* every step's slot table and the final hit / miss / eviction counts equal
  the oracle's slot policy (cache.py:410 restated);
* the per-slot outputs of sampled tokens are within tolerance of the C
  restatement of the expert FFN run on the experts read back from the host
  store (so a wrong copy, a wrong slot or a stale table all fail);
* one full SigmoidGroupMoEBlock call (router, sigmoid + correction bias,
  8 groups / top-4 groups / top-8, routed scale 2.5, shared expert) through
  the paged seam: routing bit-exact with the C oracle, output within
  tolerance.
"""

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import pmoe_oracle as O
from tests.golden.make_golden import zipf_trace
from tests.util import bits_to_bf16_tensor, check_close, slot_to_expert

pytestmark = pytest.mark.gpu

DEV = "cuda"
D, E, I, K, SLOTS = 7168, 384, 2048, 8, 96


def _store_expert(store, g, e):
    """Expert e of layer 0 of the pinned host store as an oracle Expert."""
    raw = store.expert_view(0, e)

    def comp(c, dtype, shape):
        off, nb = int(g.off[c]), int(g.nbytes[c])
        return np.ascontiguousarray(raw[off:off + nb]).view(dtype).reshape(shape)

    def qt(c0, rows, cols):
        return O.QTensor(comp(c0, np.uint32, (rows, cols * g.bits // 32)),
                         comp(c0 + 1, np.uint16, (rows, cols // 64)),
                         comp(c0 + 2, np.uint16, (rows, cols // 64)), g.bits, 64, cols)

    return O.Expert(qt(0, I, D), qt(3, I, D), qt(6, D, I))


@pytest.fixture(scope="module")
def deepseek_cache():
    from pagedmoe_amd._lib import geom
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore
    from pagedmoe_amd.slab import SlabStore

    g = geom(D, I, 4)
    print(f"[deepseek] filling a pinned store of {E} experts "
          f"({E * int(g.expert_bytes) / 1e9:.1f} GB)", flush=True)
    store = HostExpertStore(g, 1, E)
    tmp = SlabStore(g, 1, DEV, zero=False)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(1234)

    def synth(slab, slot):
        for prefix, rows, cols in (("gate_proj", I, D), ("up_proj", I, D), ("down_proj", D, I)):
            slab.quantize_into(slot, prefix,
                               torch.randn((rows, cols), generator=gen, device=DEV) * 0.02)

    for e in range(E):
        synth(tmp, 0)
        store.write_from_slot(0, e, tmp, 0)
    tmp.release()
    cache = ExpertCache(g, SLOTS, [0], E, host_store=store, n_shared=1, device=DEV)
    synth(cache.slab, cache.shared_slot(0))
    torch.cuda.synchronize()
    yield g, store, cache
    cache.close()
    store.close()


@pytest.mark.timeout(400)
def test_deepseek_zipf_paging_vs_oracle(deepseek_cache):
    from pagedmoe_amd.streaming import StreamedSwitchGLU

    g, store, cache = deepseek_cache
    st = StreamedSwitchGLU(0, None, cache)
    trace = zipf_trace(seed=0, steps=160, n_experts=E, k=K)
    pol = O.SlotPolicy(SLOTS)
    h0 = cache.stats()
    rng = np.random.default_rng(5)
    checked = {0, 1, 40, 95, 159}
    experts = {}
    print(f"[deepseek] {len(trace)} Zipf steps through a {SLOTS}-slot slab", flush=True)
    for t, ids in enumerate(trace):
        xb = O.bf16_round(rng.standard_normal((1, D), dtype=np.float32))
        ind = torch.tensor([ids], dtype=torch.int32, device=DEV)
        y = st(bits_to_bf16_tensor(xb, DEV), ind)
        pol.step(0, ids)
        assert np.array_equal(cache.host_table(0), pol.table(0, E)), t
        if t in checked:
            yf = y.float().cpu().numpy()[0]
            x = O.bf16_to_f32(xb[0])
            for j, e in enumerate(ids):
                if e not in experts:
                    experts[e] = _store_expert(store, g, e)
                ref = C.expert_ffn(experts[e], x, D, I, 4).astype(np.float64)
                check_close(yf[j], ref, f"Zipf step {t} slot {j} (expert {e})")
    s = cache.stats()
    assert (s["hits"] - h0["hits"], s["misses"] - h0["misses"],
            s["evictions"] - h0["evictions"]) == (pol.hits, pol.misses, pol.evictions)
    assert pol.evictions > 0 and 0.3 < pol.hits / (pol.hits + pol.misses) < 0.95
    # the resident slots hold the host store's bytes
    table = cache.host_table(0)
    for e in [int(i) for i in np.flatnonzero(table >= 0)[:6]]:
        got = cache.slab.slot_bytes(int(table[e])).cpu().numpy()
        assert np.array_equal(got, store.expert_view(0, e)), e


@pytest.mark.timeout(200)
def test_deepseek_block_routing_and_output_vs_oracle(deepseek_cache):
    from pagedmoe_amd.streaming import SigmoidGroupMoEBlock, StreamedSwitchGLU

    g, store, cache = deepseek_cache
    rng = np.random.default_rng(6)
    gwb = O.bf16_round(rng.standard_normal((E, D), dtype=np.float32) * np.float32(0.02))
    bias = (rng.standard_normal(E, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    st = StreamedSwitchGLU(0, None, cache)
    blk = SigmoidGroupMoEBlock(bits_to_bf16_tensor(gwb, DEV), torch.from_numpy(bias).to(DEV), st,
                               top_k=K, n_group=8, topk_group=4, routed_scaling_factor=2.5)
    shared = slot_to_expert(cache.slab, cache.shared_slot(0))
    for step in range(3):
        xb = O.bf16_round(rng.standard_normal((1, D), dtype=np.float32))
        out = blk(bits_to_bf16_tensor(xb, DEV)).float().cpu().numpy()[0]
        gi, gw = blk.last_routing
        ref_i, ref_w = C.sigmoid_group_topk(C.router_logits(xb, gwb), bias, 8, 4, K, True, 2.5)
        assert np.array_equal(gi.cpu().numpy(), ref_i), step
        assert np.array_equal(gw.cpu().numpy(), ref_w), step
        x = O.bf16_to_f32(xb[0])
        acc = C.expert_ffn(shared, x, D, I, 4).astype(np.float64)
        for j in range(K):
            ex = _store_expert(store, g, int(ref_i[0, j]))
            acc += np.float64(ref_w[0, j]) * C.expert_ffn(ex, x, D, I, 4).astype(np.float64)
        check_close(out, acc, f"DeepSeek-shaped block step {step}")
