"""ctypes loader for the oracle's C restatement (test infrastructure only)."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "_build" / "libpmoe_oracle.so"
_lib = None


class PmoExpert(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p * 3), ("s", ctypes.c_void_p * 3), ("b", ctypes.c_void_p * 3)]


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise FileNotFoundError(f"{LIB} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(str(LIB))
        _lib.pmo_scratch_floats.restype = ctypes.c_size_t
        _lib.pmo_threads.restype = ctypes.c_int
        _lib.pmo_pexp.restype = ctypes.c_float
        _lib.pmo_pexp.argtypes = [ctypes.c_float]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def router_logits(x_bits, w_bits, bias=None):
    x = np.ascontiguousarray(x_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    n, d = x.shape
    e = w.shape[0]
    out = np.empty((n, e), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().pmo_router_logits(_p(x), _p(w), None if b is None else _p(b), n, d, e, _p(out))
    return out


def softmax_topk(logits, k, norm=True):
    l = np.ascontiguousarray(logits, np.float32)
    n, e = l.shape
    inds = np.empty((n, k), np.int32)
    w = np.empty((n, k), np.float32)
    lib().pmo_softmax_topk(_p(l), n, e, k, int(norm), _p(inds), _p(w))
    return inds, w


def sigmoid_group_topk(logits, bias, n_group, topk_group, k, norm=True, scale=1.0):
    l = np.ascontiguousarray(logits, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    n, e = l.shape
    inds = np.empty((n, k), np.int32)
    w = np.empty((n, k), np.float32)
    lib().pmo_sigmoid_group_topk(_p(l), _p(b), n, e, n_group, topk_group, k, int(norm),
                                 ctypes.c_float(scale), _p(inds), _p(w))
    return inds, w


def make_experts(experts: list):
    """experts: list of objects with .gate/.up/.down QTensor (numpy arrays,
    kept alive by the caller).  Returns a ctypes array of PmoExpert."""
    arr = (PmoExpert * len(experts))()
    for i, ex in enumerate(experts):
        for j, qt in enumerate((ex.gate, ex.up, ex.down)):
            arr[i].w[j] = qt.weight.ctypes.data
            arr[i].s[j] = qt.scales.ctypes.data
            arr[i].b[j] = qt.biases.ctypes.data
    return arr


class DecodeLayer:
    """Decode MoE layer on the host cores (the cpu_baseline port)."""

    def __init__(self, gate_w_bits, experts, hidden, inter, top_k, bits):
        self.gw = np.ascontiguousarray(gate_w_bits, np.uint16)
        self.experts = experts
        self.carr = make_experts(experts)
        self.d, self.i, self.k, self.bits = hidden, inter, top_k, bits
        self.e = len(experts)
        self.scratch = np.empty(lib().pmo_scratch_floats(hidden, inter), np.float32)

    def __call__(self, x_bits):
        x = np.ascontiguousarray(x_bits, np.uint16)
        n = x.shape[0]
        logits = np.empty((n, self.e), np.float32)
        inds = np.empty((n, self.k), np.int32)
        w = np.empty((n, self.k), np.float32)
        out = np.empty((n, self.d), np.float32)
        lib().pmo_moe_decode(_p(x), _p(self.gw), n, self.d, self.e, self.i, self.k, self.bits,
                             self.carr, _p(logits), _p(inds), _p(w), _p(out), _p(self.scratch))
        return inds, w, out


def threads() -> int:
    return int(lib().pmo_threads())


def expert_ffn(ex, x_f32, hidden, inter, bits):
    """down(silu(gate x) * (up x)) of one expert for one token, fp32 on the
    host (pmo_expert_ffn); ex has .gate/.up/.down QTensors."""
    arr = make_experts([ex])
    x = np.ascontiguousarray(x_f32, np.float32).reshape(-1)
    y = np.empty(hidden, np.float32)
    scratch = np.empty(lib().pmo_scratch_floats(hidden, inter), np.float32)
    lib().pmo_expert_ffn(arr, _p(x), hidden, inter, bits, _p(y), _p(scratch))
    return y
