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
