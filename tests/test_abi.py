"""The C ABI library loads on the CPU host and exports every symbol that
include/pmoe.h declares; host-only entry points (geometry, slot policy)
behave.  No compute call touches a GPU here."""

import ctypes
import re
from pathlib import Path

import pytest

from pagedmoe_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pmoe.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the same surface
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_abi_version():
    assert _lib.lib().pmoe_abi_version() == 1


@pytest.mark.parametrize("hidden,inter,bits,expect", [
    (1024, 512, 4, 884_736), (4096, 1536, 4, 10_616_832), (7168, 2048, 4, 24_772_608),
    (2048, 512, 6, 2_555_904)])
def test_geometry_per_expert_bytes(hidden, inter, bits, expect):
    g = _lib.geom(hidden, inter, bits)
    assert g.expert_bytes == expect
    assert sum(g.nbytes) == expect
    assert all(g.off[i] % 256 == 0 for i in range(9))
    assert g.nbytes[0] == inter * hidden * bits // 8          # gate_proj.weight
    assert g.nbytes[1] == inter * (hidden // 64) * 2          # gate_proj.scales
    assert g.nbytes[6] == hidden * inter * bits // 8          # down_proj.weight


def test_errors_are_reported():
    g = _lib.Geom()
    rc = _lib.lib().pmoe_geom_init(ctypes.byref(g), 1000, 512, 4, 64)
    assert rc == -1
    assert b"multiples of 64" in _lib.lib().pmoe_last_error()
    with pytest.raises(_lib.PmoeError):
        _lib.geom(1024, 512, 5)


def test_workspace_query_is_host_only():
    g = _lib.geom(4096, 1536, 4)
    nb = _lib.lib().pmoe_moe_workspace(ctypes.byref(g), 8, 8, 0, 128)
    assert nb > 8 * 8 * 1536 * 2 + 8 * 8 * 4096 * 4


@pytest.mark.parametrize("n", [1, 2])
@pytest.mark.parametrize("cfg", [
    dict(scoring=0, n_experts=8, top_k=9),                                  # k > E
    dict(scoring=1, n_experts=30, top_k=4, n_group=8, topk_group=4),        # E % n_group
    dict(scoring=1, n_experts=32, top_k=4, n_group=8, topk_group=9),        # topk_group > n_group
    dict(scoring=1, n_experts=32, top_k=9, n_group=8, topk_group=2),        # k > kept experts
    dict(scoring=7, n_experts=32, top_k=4),                                 # unknown scoring
])
def test_moe_block_rejects_bad_routing_before_any_launch(n, cfg):
    """pmoe_moe_block validates the routing config once, before it chooses
    the one-launch (n = 1) or three-launch (n = 2) decode; the host rejects
    it, so nothing is launched and the dummy pointers are never read."""
    lib = _lib.lib()
    g = _lib.geom(1024, 512, 4)
    rc = _lib.RouteCfg()
    rc.scoring = cfg["scoring"]
    rc.n_experts = cfg["n_experts"]
    rc.top_k = cfg["top_k"]
    rc.norm_topk_prob = 1
    rc.n_group = cfg.get("n_group", 1)
    rc.topk_group = cfg.get("topk_group", 1)
    rc.routed_scale = 1.0
    dummy = ctypes.c_void_p(0x1000)
    r = lib.pmoe_moe_block(ctypes.byref(g), ctypes.byref(rc), dummy, dummy, dummy, dummy, None,
                           dummy, n, -1, None, dummy, dummy, dummy, dummy, 1 << 30, None)
    assert r == -1, lib.pmoe_last_error()
    assert b"routing" in lib.pmoe_last_error()


def test_prefill_tile_rows_by_rows_per_expert(monkeypatch):
    """32-row prefill tiles when the routed experts see at most 32 rows each
    on average (Qwen3-Next-shaped 1024-token prefill: 11 columns x 1024
    tokens over 512 experts), 128-row tiles above (Qwen3-235B-shaped 2048-token
    prefill: 16 rows x 128 per expert); PMOE_PREFILL_SMALL pins either."""
    f = _lib.lib().pmoe_prefill_tile_rows
    monkeypatch.delenv("PMOE_PREFILL_SMALL", raising=False)
    assert f(1024, 11, 512) == 32
    assert f(2048, 8, 128) == 128
    assert f(128, 8, 32) == 32 and f(129, 8, 32) == 128   # 1024 rows vs 32 x 32
    monkeypatch.setenv("PMOE_PREFILL_SMALL", "1")
    assert f(2048, 8, 128) == 32
    monkeypatch.setenv("PMOE_PREFILL_SMALL", "0")
    assert f(1024, 11, 512) == 128
