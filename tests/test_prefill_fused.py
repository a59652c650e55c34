"""The fused prefill pass (pagedmoe_amd/prefill_fused.py) on a toy pre-norm
decoder with a KV cache, on the CPU: a long call sub-chunks attention and
runs the feed-forward block once, and gives the same outputs and the same
cache as the stock layer call (prefill_fused.py:195-245 behaviour)."""

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
    plan = PF.attention_plan(layer, 300, 0)
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
        assert layer.self_attn.calls == len(PF.attention_plan(layer, 100, offset)) > 1


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
    assert DecoderLayer.forward is not orig
    PF.uninstall()
    assert DecoderLayer.forward is orig


def test_off_switch(monkeypatch):
    monkeypatch.setattr(config, "FUSED_PREFILL", False)
    assert not PF.install(Model())
