"""ctypes binding of libpmoe.so (the C ABI declared in include/pmoe.h).

The library is built in-tree (``__graft_entry__.build()`` or ``make -C
pagedmoe_amd/csrc``).  There is no fallback: if the library is missing every
entry point raises ``PmoeError``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpmoe.so"

PMOE_OK = 0
PMOE_NCOMP = 9
COMPONENTS = (
    "gate_proj.weight", "gate_proj.scales", "gate_proj.biases",
    "up_proj.weight", "up_proj.scales", "up_proj.biases",
    "down_proj.weight", "down_proj.scales", "down_proj.biases",
)
SCORE_SOFTMAX = 0
SCORE_SIGMOID = 1


class PmoeError(RuntimeError):
    """An entry point of libpmoe returned an error (or the library is absent)."""


class Geom(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("expert_bytes", ctypes.c_int64),
        ("off", ctypes.c_int64 * PMOE_NCOMP),
        ("nbytes", ctypes.c_int64 * PMOE_NCOMP),
    ]


class RouteCfg(ctypes.Structure):
    _fields_ = [
        ("scoring", ctypes.c_int32),
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("norm_topk_prob", ctypes.c_int32),
        ("n_group", ctypes.c_int32),
        ("topk_group", ctypes.c_int32),
        ("routed_scale", ctypes.c_float),
    ]


class SlabStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "hits", "misses", "evictions", "starved", "installs", "resident", "slots",
        "budget", "reserve", "stitched", "bytes_copied", "prefill_slot_reads",
        "prefill_installs", "stage_reads", "prefill_starved", "stage_slots", "flow_admits",
        "spec_started", "spec_claims", "spec_claims_late", "spec_dropped",
        "ahead_started", "ahead_claims")]


class LedgerRec(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("kind", "who", "a", "b", "c")]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_I32P = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); every symbol include/pmoe.h declares.
SIGNATURES = {
    "pmoe_abi_version": (_I, []),
    "pmoe_last_error": (ctypes.c_char_p, []),
    "pmoe_geom_init": (_I, [ctypes.POINTER(Geom), _I, _I, _I, _I]),
    "pmoe_router_logits": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "pmoe_route_softmax_topk": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "pmoe_route_sigmoid_group_topk": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P]),
    "pmoe_dispatch_workspace": (_SZ, [_I, _I]),
    "pmoe_dispatch": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "pmoe_quantize": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "pmoe_dequant": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "pmoe_moe_workspace": (_SZ, [ctypes.POINTER(Geom), _I, _I, _I, _I]),
    "pmoe_moe_workspace_init": (_I, [_P, _SZ, _P]),
    "pmoe_moe_workspace_status": (_I, [_P, ctypes.POINTER(ctypes.c_uint32), _P]),
    "pmoe_prefill_tile_rows": (_I, [_I, _I, _I]),
    "pmoe_moe_workspace_error_async": (_I, [_P, _P, _P]),
    "pmoe_set_barrier_spin": (_I, [ctypes.c_uint64]),
    "pmoe_set_split_probe": (_I, [_I]),
    "pmoe_switch_glu": (_I, [ctypes.POINTER(Geom), _P, _P, _I, _P, _P, _I, _I, _P, _P, _SZ, _P]),
    "pmoe_moe_experts": (_I, [ctypes.POINTER(Geom), _P, _P, _I, _P, _P, _P, _I, _I, _I, _P,
                              _P, _P, _SZ, _P]),
    "pmoe_moe_block": (_I, [ctypes.POINTER(Geom), ctypes.POINTER(RouteCfg), _P, _P, _P, _P, _P,
                            _P, _I, _I, _P, _P, _P, _P, _P, _SZ, _P]),
    "pmoe_moe_block_noalloc": (_I, [ctypes.POINTER(Geom), ctypes.POINTER(RouteCfg), _P, _P, _P,
                                    _P, _P, _P, _I, _I, _P, _P, _P, _P, _P]),
    "pmoe_combine": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _P]),
    "pmoe_count_missing": (_I, [_P, _P, _I, _I, _P, _P]),
    "pmoe_slab_create": (_I, [ctypes.POINTER(_P), _I, _I, _I, _F, _I, _I]),
    "pmoe_slab_destroy": (_I, [_P]),
    "pmoe_slab_device_table": (_P, [_P, _I]),
    "pmoe_slab_host_table": (_I, [_P, _I, _I32P]),
    "pmoe_slab_request": (_I, [_P, _I, _I32P, _I, _I32P, _I32P, ctypes.POINTER(_I)]),
    "pmoe_slab_stitch": (_I, [_P]),
    "pmoe_slab_publish": (_I, [_P, _I, _P]),
    "pmoe_slab_sync_table": (_I, [_P, _I, _P]),
    "pmoe_slab_dirty": (_I, [_P, _I]),
    "pmoe_slab_read_device_row": (_I, [_P, _I, _I32P]),
    "pmoe_slab_admit": (_I, [_P, _I, _I32P, _I, _I32P, _I32P, ctypes.POINTER(_I), _I]),
    "pmoe_slab_install": (_I, [_P, _I, _I32P, _I]),
    "pmoe_slab_set_spec_engine": (_I, [_P, _P]),
    "pmoe_slab_speculate": (_I, [_P, ctypes.POINTER(Geom), _P, _P, _I, _I32P, _I, _I,
                                 ctypes.POINTER(_I)]),
    "pmoe_slab_drop_staged": (_I, [_P]),
    "pmoe_slab_prefill_ahead": (_I, [_P, ctypes.POINTER(Geom), _P, _P, _I, _I32P, _I, _I, _I,
                                     ctypes.POINTER(_I)]),
    "pmoe_slab_set_stage": (_I, [_P, _I, _I]),
    "pmoe_slab_capacity": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "pmoe_slab_prefill_request": (_I, [_P, _I, _I32P, _I, _I32P, _I32P, ctypes.POINTER(_I),
                                       ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "pmoe_slab_prefill_publish": (_I, [_P, _I, _P]),
    "pmoe_slab_prefill_done": (_I, [_P, _I]),
    "pmoe_slab_stats_get": (_I, [_P, ctypes.POINTER(SlabStats)]),
    "pmoe_host_alloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "pmoe_host_free": (_I, [_P]),
    "pmoe_copy_engine_create": (_I, [ctypes.POINTER(_P), _SZ, _I]),
    "pmoe_copy_engine_destroy": (_I, [_P]),
    "pmoe_copy_submit": (_I, [_P, _P, _P, _SZ, _I]),
    "pmoe_copy_flush": (_I, [_P, _P]),
    "pmoe_copy_fence": (_I, [_P, _P]),
    "pmoe_copy_issue": (_I, [_P, ctypes.POINTER(_I)]),
    "pmoe_copy_batch_done": (_I, [_P, _I]),
    "pmoe_copy_batch_join": (_I, [_P, _I, _P]),
    "pmoe_copy_batch_wait": (_I, [_P, _I]),
    "pmoe_copy_batch_release": (_I, [_P, _I]),
    "pmoe_copy_join": (_I, [_P, _P]),
    "pmoe_copy_sync": (_I, [_P]),
    "pmoe_copy_bytes": (ctypes.c_int64, [_P]),
    "pmoe_slab_fetch": (_I, [_P, _P, ctypes.POINTER(Geom), _P, _P, _I, _I32P, _I,
                             ctypes.POINTER(_I), _P]),
    "pmoe_slab_fetch_prefill": (_I, [_P, _P, ctypes.POINTER(Geom), _P, _P, _I, _I32P, _I,
                                     ctypes.POINTER(_I), ctypes.POINTER(_I),
                                     ctypes.POINTER(_I)]),
    "pmoe_ledger_enable": (_I, [_I]),
    "pmoe_ledger_note": (_I, [ctypes.c_int64, _P, ctypes.c_int64, ctypes.c_int64,
                              ctypes.c_int64]),
    "pmoe_ledger_drain": (_I, [ctypes.POINTER(LedgerRec), _I, ctypes.POINTER(_I)]),
    "pmoe_probe_sink_bytes": (_SZ, []),
    "pmoe_probe_read": (_I, [_P, _SZ, _P, _SZ, _P]),
    "pmoe_probe_copy": (_I, [_P, _P, _SZ, _P]),
    "pmoe_profile_begin": (_I, [_I]),
    "pmoe_profile_end": (_I, []),
    "pmoe_profile_kernels": (_I, []),
    "pmoe_profile_name": (ctypes.c_char_p, [_I]),
    "pmoe_profile_read": (_I, [_I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises PmoeError when it has not been built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("PMOE_LIB", LIB_PATH))
        if not path.exists():
            raise PmoeError(
                f"libpmoe.so not found at {path}: build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`make -C pagedmoe_amd/csrc`")
        handle = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str = "") -> None:
    """Raise PmoeError with the library's message for a nonzero status."""
    if rc != PMOE_OK:
        msg = lib().pmoe_last_error().decode(errors="replace")
        raise PmoeError(f"{what or 'pmoe'} failed ({rc}): {msg}")


def geom(hidden: int, inter: int, bits: int, group: int = 64) -> Geom:
    g = Geom()
    check(lib().pmoe_geom_init(ctypes.byref(g), hidden, inter, bits, group), "pmoe_geom_init")
    return g


class KernelTimer:
    """Context manager: per-kernel HIP-event time of every libpmoe launch in
    the block (pmoe_profile_*).  ``result`` maps kernel name ->
    (total_ms, launches)."""

    def __init__(self, capacity: int = 65536):
        self.capacity = capacity
        self.result: dict = {}

    def __enter__(self):
        check(lib().pmoe_profile_begin(self.capacity), "pmoe_profile_begin")
        return self

    def __exit__(self, *exc):
        L = lib()
        check(L.pmoe_profile_end(), "pmoe_profile_end")
        for k in range(L.pmoe_profile_kernels()):
            ms = ctypes.c_double()
            cnt = ctypes.c_int64()
            check(L.pmoe_profile_read(k, ctypes.byref(ms), ctypes.byref(cnt)), "pmoe_profile_read")
            if cnt.value:
                self.result[L.pmoe_profile_name(k).decode()] = (ms.value, cnt.value)
        return False
