"""GPU: pmoe_moe_block_noalloc, the MoE block entry point that allocates
nothing (its workspace is the library's static per-GPU scratch array),
called through the C ABI and checked against pmoe_moe_block with a caller
workspace on the same inputs: routing ids and weights bit-exact, layer
outputs bit-identical (the same kernels run; only the workspace differs).
Two calls in a row on the same scratch, the second with fewer tokens, for
each configuration; a prefill-sized call is refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import pmoe_oracle as O
from tests.util import bits_to_bf16_tensor, fill_slab_gpu

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _lib():
    from pagedmoe_amd import _lib
    return _lib


class _Layer:
    def __init__(self, hidden, experts, inter, top_k, bits=4, scoring="softmax", shared=False,
                 shared_gate=False, n_group=1, topk_group=1, scale=1.0, seed=0):
        from pagedmoe_amd import kernels as K
        from pagedmoe_amd._lib import geom
        from pagedmoe_amd.slab import SlabStore
        self.g = geom(hidden, inter, bits)
        n_slots = experts + int(shared)
        self.slab = SlabStore(self.g, n_slots, DEV)
        fill_slab_gpu(self.slab, range(n_slots), seed=seed)
        rng = np.random.default_rng(seed)
        self.gate = bits_to_bf16_tensor(O.bf16_round(
            rng.standard_normal((experts, hidden), dtype=np.float32) * np.float32(0.02)), DEV)
        self.table = torch.arange(experts, dtype=torch.int32, device=DEV)
        self.rc = K.route_cfg(scoring, experts, top_k, True, n_group, topk_group, scale)
        self.bias = None
        if scoring == "sigmoid":
            self.bias = torch.from_numpy((rng.standard_normal(experts, dtype=np.float32)
                                          * np.float32(0.1)).astype(np.float32)).to(DEV)
        self.shared_slot = experts if shared else -1
        self.sgate = None
        if shared_gate:
            self.sgate = bits_to_bf16_tensor(O.bf16_round(
                rng.standard_normal((1, hidden), dtype=np.float32) * np.float32(0.02)), DEV)
        self.hidden, self.k = hidden, top_k

    def x(self, n, seed):
        rng = np.random.default_rng(seed)
        return bits_to_bf16_tensor(O.bf16_round(rng.standard_normal((n, self.hidden),
                                                                    dtype=np.float32)), DEV)

    def _outs(self, n):
        return (torch.empty((n, self.hidden), dtype=torch.bfloat16, device=DEV),
                torch.empty((n, self.k), dtype=torch.int32, device=DEV),
                torch.empty((n, self.k), dtype=torch.float32, device=DEV))

    def _common(self, x):
        p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
        return (ctypes.byref(self.g), ctypes.byref(self.rc), p(self.slab.buf), p(self.table),
                p(self.gate), p(self.bias), None, p(x), x.shape[0], self.shared_slot,
                p(self.sgate))

    def with_workspace(self, x):
        from pagedmoe_amd import kernels as K
        L = _lib()
        out, inds, w = self._outs(x.shape[0])
        ws = K.moe_workspace(self.g, x.shape[0], self.k, int(self.shared_slot >= 0),
                             self.rc.n_experts, DEV, fresh=True)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        L.check(L.lib().pmoe_moe_block(*self._common(x), ctypes.c_void_p(out.data_ptr()),
                                       ctypes.c_void_p(inds.data_ptr()),
                                       ctypes.c_void_p(w.data_ptr()),
                                       ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream),
                "pmoe_moe_block")
        return out, inds, w

    def noalloc(self, x):
        L = _lib()
        out, inds, w = self._outs(x.shape[0])
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        L.check(L.lib().pmoe_moe_block_noalloc(*self._common(x), ctypes.c_void_p(out.data_ptr()),
                                               ctypes.c_void_p(inds.data_ptr()),
                                               ctypes.c_void_p(w.data_ptr()), stream),
                "pmoe_moe_block_noalloc")
        return out, inds, w


CONFIGS = {
    # Qwen3-235B-shaped decode: 8 tokens (three-launch decode), then 1 (one launch)
    "qwen3-235b": (dict(hidden=4096, experts=128, inter=1536, top_k=8), (8, 1)),
    # DeepSeek-style routing with a shared expert at small dims: 6 tokens, then 2
    "sigmoid-shared": (dict(hidden=1024, experts=64, inter=512, top_k=6, scoring="sigmoid",
                            shared=True, n_group=8, topk_group=4, scale=2.5), (6, 2)),
    # DeepSeek-V3-style top-8 with a shared expert: 2 tokens (three-launch decode),
    # then 1 (router launch, then the given-ids expert-per-XCD launch)
    "sigmoid-shared-top8": (dict(hidden=1024, experts=64, inter=512, top_k=8, scoring="sigmoid",
                                 shared=True, n_group=8, topk_group=4, scale=2.5), (2, 1)),
    # Qwen3-Next-style: 6-bit, top-10 of 512 plus a gated shared expert: 8, then 1
    "qwen3-next-6bit": (dict(hidden=2048, experts=512, inter=512, top_k=10, bits=6, shared=True,
                             shared_gate=True), (8, 1)),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_noalloc_matches_moe_block_on_two_calls(name):
    cfg, sizes = CONFIGS[name]
    layer = _Layer(seed=3, **cfg)
    for call, n in enumerate(sizes):
        print(f"[noalloc] {name} call {call} n={n}", flush=True)
        x = layer.x(n, seed=10 + call)
        ref = layer.with_workspace(x)
        got = layer.noalloc(x)
        torch.cuda.synchronize()
        assert torch.equal(got[1], ref[1]), f"{name} call {call}: routing ids differ"
        assert torch.equal(got[2], ref[2]), f"{name} call {call}: routing weights differ"
        assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16)), \
            f"{name} call {call}: layer outputs differ"
        assert torch.isfinite(got[0].float()).all()


def test_noalloc_refuses_prefill_sized_calls():
    """2048 tokens need far more than the 32 MiB static scratch: the host
    refuses with PMOE_ESPACE and a message naming the sizes; nothing runs."""
    from pagedmoe_amd import _lib as L
    g = L.geom(4096, 1536, 4)
    from pagedmoe_amd import kernels as K
    rc = K.route_cfg("softmax", 128, 8)
    dummy = ctypes.c_void_p(0x1000)
    r = L.lib().pmoe_moe_block_noalloc(ctypes.byref(g), ctypes.byref(rc), dummy, dummy, dummy,
                                       None, None, dummy, 2048, -1, None, dummy, dummy, dummy,
                                       None)
    assert r == -5
    msg = L.lib().pmoe_last_error().decode()
    assert "static scratch holds 33554432" in msg, msg
