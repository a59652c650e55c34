"""The fused prefill pass (pagedmoe_amd/prefill_fused.py) on toy decoders
with a KV cache, on the CPU: a long call splits attention and runs the
feed-forward block once, and gives the same outputs and the same cache as the
stock layer call (reference prefill_fused.py:195-245 and :248-307
behaviour).  Hybrid stacks whose linear-attention instances share a class
with full-attention ones keep the stock call on those instances."""

import math

import pytest
import torch
from torch import nn

from pagedmoe_amd import config, prefill_fused as PF


class KVCache:
    """Per-layer cache with the reference's interface: offset = keys held."""

    def __init__(self):
        self.k = None
        self.v = None

    @property
    def offset(self):
        return 0 if self.k is None else self.k.shape[2]

    def update_and_fetch(self, k, v):
        self.k = k if self.k is None else torch.cat([self.k, k], dim=2)
        self.v = v if self.v is None else torch.cat([self.v, v], dim=2)
        return self.k, self.v


class Attention(nn.Module):
    def __init__(self, d, heads, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.n_heads = heads
        self.wq, self.wk, self.wv, self.wo = (nn.Parameter(torch.randn(d, d, generator=g,
                                                                       dtype=torch.float64) / d ** 0.5)
                                              for _ in range(4))
        self.calls = 0

    def forward(self, x, mask, cache):
        self.calls += 1
        b, t, d = x.shape
        h = self.n_heads
        q, k, v = (z.reshape(b, t, h, d // h).transpose(1, 2) for z in (x @ self.wq, x @ self.wk,
                                                                        x @ self.wv))
        k, v = cache.update_and_fetch(k, v)
        s = q @ k.transpose(-1, -2) / math.sqrt(d // h)
        if mask is not None:
            s = s + mask
        o = torch.softmax(s, dim=-1) @ v
        return o.transpose(1, 2).reshape(b, t, d) @ self.wo


class RMSNorm(nn.Module):
    def forward(self, x):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)


class CountingMLP(nn.Module):
    def __init__(self, d, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed + 100)
        self.w = nn.Parameter(torch.randn(d, d, generator=g, dtype=torch.float64) / d ** 0.5)
        self.calls = []

    def forward(self, x):
        self.calls.append(x.shape[1])
        return torch.tanh(x @ self.w)


class DecoderLayer(nn.Module):
    def __init__(self, d, heads, seed):
        super().__init__()
        self.self_attn = Attention(d, heads, seed)
        self.input_layernorm = RMSNorm()
        self.post_attention_layernorm = RMSNorm()
        self.mlp = CountingMLP(d, seed)

    def forward(self, x, mask=None, cache=None):
        h = x + self.self_attn(self.input_layernorm(x), mask, cache)
        return h + self.mlp(self.post_attention_layernorm(h))


class Model(nn.Module):
    def __init__(self, d=64, heads=4, n_layers=2):
        super().__init__()
        self.layers = nn.ModuleList([DecoderLayer(d, heads, s) for s in range(n_layers)])

    def forward(self, x, caches):
        t, off = x.shape[1], caches[0].offset
        q = torch.arange(off, off + t)[:, None]
        k = torch.arange(off + t)[None, :]
        mask = torch.where(k <= q, 0.0, float("-inf")).to(torch.float64)
        for layer, c in zip(self.layers, caches):
            x = layer(x, mask, c)
        return x


@pytest.fixture
def fused(monkeypatch):
    monkeypatch.setattr(config, "FUSED_PREFILL", True)
    monkeypatch.setattr(config, "ATTN_SUB_CHUNK", 24)
    monkeypatch.setattr(config, "ATTN_SCORE_MB", 1024)
    yield
    PF.uninstall()


def test_attention_plan_covers_and_shrinks_with_kv(monkeypatch):
    monkeypatch.setattr(config, "ATTN_SUB_CHUNK", 4096)
    monkeypatch.setattr(config, "ATTN_SCORE_MB", 1)      # 1 MiB of fp32 scores
    layer = DecoderLayer(64, 4, 0)
    plan = PF.row_splits(layer, 300, 0)
    assert plan[0][0] == 0 and plan[-1][1] == 300
    assert all(a[1] == b[0] for a, b in zip(plan, plan[1:]))
    sizes = [e - s for s, e in plan]
    assert sizes == sorted(sizes, reverse=True) and sizes[-1] < sizes[0]
    kv = 0
    for s, e in plan:   # every sub-chunk's scores fit the budget
        assert 4 * 4 * (e - s) * (kv + e - s) <= 1 << 20 or e - s == 1
        kv += e - s


@pytest.mark.parametrize("offset", [0, 40])
def test_fused_layer_equals_stock_and_runs_mlp_once(fused, offset):
    torch.manual_seed(0)
    stock, fused_m = Model(), Model()
    fused_m.load_state_dict(stock.state_dict())
    cs, cf = [KVCache(), KVCache()], [KVCache(), KVCache()]
    if offset:   # a cache that already holds `offset` keys
        pre = torch.randn(1, offset, 64, dtype=torch.float64)
        stock(pre, cs)
        fused_m(pre, cf)
    assert PF.install(fused_m)
    x = torch.randn(1, 100, 64, dtype=torch.float64)
    for layer in fused_m.layers:
        layer.self_attn.calls = 0
        layer.mlp.calls.clear()
    ys = stock(x, cs)
    yf = fused_m(x, cf)
    assert torch.allclose(yf, ys, rtol=1e-10, atol=1e-10)
    for a, b in zip(cs, cf):
        assert torch.allclose(a.k, b.k, rtol=1e-12, atol=1e-12) and a.offset == b.offset
    for layer in fused_m.layers:
        assert layer.mlp.calls == [100]                 # the MoE ran once, over every token
        assert layer.self_attn.calls == len(PF.row_splits(layer, 100, offset)) > 1


def test_short_calls_take_the_stock_path(fused):
    m = Model()
    assert PF.install(m)
    cache = [KVCache(), KVCache()]
    m(torch.randn(1, 8, 64, dtype=torch.float64), cache)
    assert all(layer.self_attn.calls == 1 for layer in m.layers)


def test_install_is_idempotent_and_uninstall_restores(fused):
    m = Model()
    orig = DecoderLayer.forward
    assert PF.install(m) and PF.install(m)
    assert DecoderLayer.forward is orig                  # the class is never touched
    assert all("forward" in layer.__dict__ and PF.installed(layer) for layer in m.layers)
    PF.uninstall(m)
    assert all("forward" not in layer.__dict__ for layer in m.layers)
    assert not any(PF.installed(layer) for layer in m.layers)


def test_rows_for_budget_is_the_largest_fitting_split():
    """Closed form against brute force: the largest c <= cap with
    4 * heads * c * (kv + c) <= budget, and at least 1."""
    for heads in (1, 3, 8):
        for kv in (0, 1, 7, 100, 5000):
            for budget in (1, 64, 4096, 1 << 20, 3 << 22):
                for cap in (1, 5, 64, 100000):
                    want = 1
                    for c in range(1, min(cap, 3000) + 1):
                        if 4 * heads * c * (kv + c) <= budget:
                            want = c
                    if cap > 3000 and 4 * heads * 3000 * (kv + 3000) <= budget:
                        continue                          # beyond the brute-force range
                    assert PF.rows_for_budget(heads, kv, budget, cap) == want, (heads, kv, budget, cap)


class LinearMixer(nn.Module):
    """A recurrent mixer standing in for a Gated DeltaNet: each row's output
    depends on every earlier row of the call (a running mean), so splitting
    its call would change the result."""

    def __init__(self):
        super().__init__()
        self.calls = []

    def forward(self, x, mask, cache):
        self.calls.append(x.shape[1])
        steps = torch.arange(1, x.shape[1] + 1, dtype=x.dtype)[None, :, None]
        return torch.cumsum(x, dim=1) / steps


class HybridLayer(nn.Module):
    """One class for both kinds, as Qwen3-Next builds them: full attention
    (self_attn) or linear attention (linear_attn, layer_type marker)."""

    def __init__(self, d, heads, seed, linear):
        super().__init__()
        if linear:
            self.linear_attn = LinearMixer()
            self.layer_type = "linear_attention"
        else:
            self.self_attn = Attention(d, heads, seed)
        self.input_layernorm = RMSNorm()
        self.post_attention_layernorm = RMSNorm()
        self.mlp = CountingMLP(d, seed)

    def forward(self, x, mask=None, cache=None):
        mixer = self.linear_attn if hasattr(self, "linear_attn") else self.self_attn
        h = x + mixer(self.input_layernorm(x), mask, cache)
        return h + self.mlp(self.post_attention_layernorm(h))


def test_hybrid_class_keeps_linear_instances_stock(fused):
    """Linear and full attention instances of one class: only the full ones
    split; a linear instance sees its whole sequence in one call (no
    AttributeError for its missing self_attn), and every output and cache
    equals the stock model's."""
    torch.manual_seed(1)
    kinds = [True, False, True, False]

    def build():
        m = Model()
        m.layers = nn.ModuleList([HybridLayer(64, 4, s, lin) for s, lin in enumerate(kinds)])
        return m

    stock, fused_m = build(), build()
    fused_m.load_state_dict(stock.state_dict())
    assert PF.install(fused_m)
    assert [PF.installed(layer) for layer in fused_m.layers] == [not k for k in kinds]
    assert [PF.layer_shape(layer) for layer in fused_m.layers] == [
        None if k else "pre_norm" for k in kinds]
    cs, cf = [KVCache() for _ in kinds], [KVCache() for _ in kinds]
    x = torch.randn(1, 100, 64, dtype=torch.float64)
    ys = stock(x, cs)
    yf = fused_m(x, cf)
    assert torch.allclose(yf, ys, rtol=1e-10, atol=1e-10)
    for layer, lin in zip(fused_m.layers, kinds):
        assert layer.mlp.calls == [100]
        if lin:
            assert layer.linear_attn.calls == [100]
        else:
            assert layer.self_attn.calls == len(PF.row_splits(layer, 100, 0)) > 1
    for a, b, lin in zip(cs, cf, kinds):
        if not lin:
            assert torch.allclose(a.k, b.k, rtol=1e-12, atol=1e-12)


def test_layers_without_a_feed_forward_keep_the_stock_call(fused):
    m = Model()
    del m.layers[1].mlp
    m.layers[1].mlp = None
    assert PF.install(m)
    assert PF.installed(m.layers[0]) and not PF.installed(m.layers[1])


class HyperConnection(nn.Module):
    """n parallel residual streams (h is [B, T, n*D]): mixes them into the
    block input x, keeps a carried residual, and an injection weight per
    stream for the block's output."""

    def __init__(self, d, n, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.d, self.n = d, n
        self.mix = nn.Parameter(torch.randn(n, generator=g, dtype=torch.float64))
        self.inj = nn.Parameter(torch.randn(n * d, n, generator=g, dtype=torch.float64) / d)

    def forward(self, h):
        streams = h.unflatten(-1, (self.n, self.d))
        x = (streams * self.mix[:, None]).sum(-2)
        inject = torch.tanh(h @ self.inj)
        return x, 0.5 * h, inject


class HyperAttention(Attention):
    def forward(self, x, rope, mask, cache, idx_cache):
        assert rope == "rope" and idx_cache == "idx"
        return super().forward(x, mask, cache)


class HyperLayer(nn.Module):
    """A hyper-connection decoder block with the positional call
    (h, rope, mask, conv_mask, cache, idx_cache, ids, prev_ctx)."""

    def __init__(self, d, n, heads, seed):
        super().__init__()
        self.self_attn = HyperAttention(d, heads, seed)
        self.mlp = CountingMLP(d, seed)
        self.attn_hyper_connection = HyperConnection(d, n, seed + 1)
        self.mlp_hyper_connection = HyperConnection(d, n, seed + 2)

    def forward(self, h, rope=None, mask=None, conv_mask=None, cache=None, idx_cache=None,
                ids=None, prev_ctx=None):
        x, carry, inject = self.attn_hyper_connection(h)
        x = self.self_attn(x, rope, mask, cache, idx_cache)
        h = carry + (x[..., None, :] * inject[..., None]).reshape(*x.shape[:-1], -1)
        x, carry, inject = self.mlp_hyper_connection(h)
        x = self.mlp(x)
        return carry + (x[..., None, :] * inject[..., None]).reshape(*x.shape[:-1], -1)


def test_hyper_connection_layer_splits_attention_only(fused):
    torch.manual_seed(2)
    d, n = 64, 2

    def build():
        m = nn.Module()
        m.layers = nn.ModuleList([HyperLayer(d, n, 4, s) for s in range(2)])
        return m

    stock, fused_m = build(), build()
    fused_m.load_state_dict(stock.state_dict())
    assert PF.install(fused_m)
    assert all(PF.layer_shape(layer) == "hyper" for layer in fused_m.layers)

    def run(m, h, caches):
        t, off = h.shape[1], caches[0].offset
        q = torch.arange(off, off + t)[:, None]
        mask = torch.where(torch.arange(off + t)[None, :] <= q, 0.0,
                           float("-inf")).to(torch.float64)
        for layer, c in zip(m.layers, caches):
            h = layer(h, "rope", mask, None, c, "idx")
        return h

    h = torch.randn(1, 90, n * d, dtype=torch.float64)
    cs, cf = [KVCache(), KVCache()], [KVCache(), KVCache()]
    ys, yf = run(stock, h, cs), run(fused_m, h, cf)
    assert torch.allclose(yf, ys, rtol=1e-10, atol=1e-10)
    for layer in fused_m.layers:
        assert layer.mlp.calls == [90]
        assert layer.self_attn.calls == len(PF.row_splits(layer, 90, 0)) > 1
    # short calls and keyword extras take the stock call
    short = torch.randn(1, 4, n * d, dtype=torch.float64)
    run(fused_m, short, cf)
    assert all(layer.mlp.calls == [90, 4] for layer in fused_m.layers)


def test_off_switch(monkeypatch):
    monkeypatch.setattr(config, "FUSED_PREFILL", False)
    assert not PF.install(Model())
