"""Expert byte ranges of safetensors checkpoints, read straight into slot layout.

Counterpart of the reference's ``safetensors_index.py`` (header parsing,
``TensorLoc``, stacked vs per-expert locators: safetensors_index.py:61-159)
and ``_layer_layout`` (streaming.py:2529-2572).  A quantized MoE checkpoint
stores each layer's experts either stacked, one tensor per component

    <prefix>.layers.<L>.mlp.switch_mlp.gate_proj.weight   [E, out, in*bits/32] u32
    <prefix>.layers.<L>.mlp.switch_mlp.gate_proj.scales   [E, out, in/64]      bf16
    ...

or per expert (``<parent>.experts.<e>.gate_proj.weight`` ...).  Either way
expert e of a component is one contiguous byte range found from the file
header alone, so an expert is read with nine ``pread`` calls straight into the
slot layout of the slab and the pinned host store (``pmoe_geom`` offsets:
gate/up/down weight, scales, biases) -- no conversion, the checkpoint on disk
stays as it is.  The u32 weight words and bf16 scale/bias rows are the
layout the kernels read (row-major per expert), so the bytes are copied
unchanged.
"""

from __future__ import annotations

import glob
import json
import os
import re
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from ._lib import COMPONENTS, Geom, PmoeError

_ITEMSIZE = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4, "I16": 2,
             "I8": 1, "U8": 1, "U32": 4, "U16": 2, "BOOL": 1}
_PROJS = ("gate_proj", "up_proj", "down_proj")
_COMPS = ("weight", "scales", "biases")


@dataclass(frozen=True)
class TensorLoc:
    """Where one tensor lives: file, dtype string, shape, absolute byte
    offset of its first element and its size (safetensors_index.py:61-89)."""

    file: str
    dtype: str
    shape: tuple
    offset: int
    nbytes: int

    def expert_slice(self, e: int) -> "TensorLoc":
        """experts[e] of a stacked [E, ...] tensor: one contiguous range."""
        n = self.shape[0]
        if not 0 <= e < n:
            raise IndexError(f"expert {e} outside a stack of {n}")
        stride = self.nbytes // n
        return TensorLoc(self.file, self.dtype, tuple(self.shape[1:]), self.offset + e * stride,
                         stride)


def read_headers(model_dir) -> dict:
    """Every tensor of ``model*.safetensors`` in model_dir -> TensorLoc.

    The format: an 8-byte little-endian header size, that many bytes of JSON
    ({name: {dtype, shape, data_offsets: [begin, end]}}, offsets relative to
    the end of the header), then the raw data (safetensors_index.py:134-159)."""
    files = sorted(glob.glob(str(Path(model_dir) / "model*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no model*.safetensors in {model_dir}")
    index = {}
    for path in files:
        with open(path, "rb") as f:
            (hsize,) = struct.unpack("<Q", f.read(8))
            header = json.loads(f.read(hsize))
        start = 8 + hsize
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            begin, end = meta["data_offsets"]
            shape = tuple(int(s) for s in meta["shape"])
            loc = TensorLoc(path, meta["dtype"], shape, start + int(begin), int(end) - int(begin))
            n = int(np.prod(shape, dtype=np.int64)) * _ITEMSIZE.get(loc.dtype, 0)
            if _ITEMSIZE.get(loc.dtype) and n != loc.nbytes:
                raise ValueError(f"{path}: {name} has {loc.nbytes} bytes for shape {shape} "
                                 f"{loc.dtype}")
            index[name] = loc
    return index


class ExpertLayout:
    """The nine components of one MoE layer: component name
    ("gate_proj.weight" ...) -> a stacked TensorLoc or {expert: TensorLoc}."""

    def __init__(self, path: str, parts: dict):
        self.path = path
        self.parts = parts

    @property
    def stacked(self) -> bool:
        return all(isinstance(v, TensorLoc) for v in self.parts.values())

    @property
    def n_experts(self) -> int:
        v = self.parts["gate_proj.weight"]
        return v.shape[0] if isinstance(v, TensorLoc) else len(v)

    def loc(self, name: str, e: int) -> TensorLoc:
        v = self.parts[name]
        if isinstance(v, TensorLoc):
            return v.expert_slice(e)
        if e not in v:
            raise KeyError(f"{self.path}: no tensor for expert {e} of {name}")
        return v[e]

    def geometry(self, group: int = 64):
        """(hidden, inter, bits) from the gate projection's shapes:
        weight [.., inter, hidden*bits/32], scales [.., inter, hidden/group]."""
        w = self.loc("gate_proj.weight", 0)
        s = self.loc("gate_proj.scales", 0)
        inter = w.shape[0]
        hidden = s.shape[1] * group
        bits, rem = divmod(w.shape[1] * 32, hidden)
        if rem or bits not in (2, 3, 4, 5, 6, 8):
            raise ValueError(f"{self.path}: weight {w.shape} / scales {s.shape} give no bit width")
        return hidden, inter, bits


def layer_layout(path: str, index: dict) -> ExpertLayout:
    """Locate one layer's expert tensors under module path ``path`` (the
    SwitchGLU, e.g. ``model.layers.3.mlp.switch_mlp``): stacked
    ``<path>.<proj>.<comp>`` first, else per-expert
    ``<parent>.experts.<e>.<proj>.<comp>`` (streaming.py:2529-2572)."""
    parts = {}
    for proj in _PROJS:
        for comp in _COMPS:
            loc = index.get(f"{path}.{proj}.{comp}")
            if loc is not None:
                parts[f"{proj}.{comp}"] = loc
    if not parts:
        parent = path.rsplit(".", 1)[0]
        pat = re.compile(re.escape(parent) + r"\.experts\.(\d+)\.(\w+)\.(weight|scales|biases)$")
        for name, loc in index.items():
            m = pat.match(name)
            if m and m.group(2) in _PROJS:
                parts.setdefault(f"{m.group(2)}.{m.group(3)}", {})[int(m.group(1))] = loc
    missing = [c for c in COMPONENTS if c not in parts]
    if missing:
        raise KeyError(f"{path}: checkpoint lacks {missing} (quantized experts with scales "
                       "and biases are required)")
    return ExpertLayout(path, parts)


_LAYER_RE = re.compile(r"^(.*\.layers\.(\d+)\.mlp)\.(?:switch_mlp\.gate_proj\.weight|"
                       r"experts\.0\.gate_proj\.weight)$")


def find_moe_layers(index: dict) -> list:
    """[(layer number, switch path)] of every MoE layer, ascending -- the
    checkpoint-side equivalent of find_switch_glus (streaming.py:2512-2526)."""
    found = {}
    for name in index:
        m = _LAYER_RE.match(name)
        if m:
            found[int(m.group(2))] = m.group(1) + ".switch_mlp"
    return sorted(found.items())


def check_layout(layout: ExpertLayout, g: Geom) -> None:
    """Every component of every expert has the slot's dtype and byte count."""
    from .slab import component_specs

    specs = component_specs(g)
    want_dtype = {"weight": ("U32", "I32"), "scales": ("BF16",), "biases": ("BF16",)}
    for c, name in enumerate(COMPONENTS):
        shape, _, nbytes, _ = specs[name]
        kind = name.split(".")[1]
        for e in range(layout.n_experts):
            loc = layout.loc(name, e)
            if loc.dtype not in want_dtype[kind]:
                raise PmoeError(f"{layout.path}: {name} is {loc.dtype}; the slab holds "
                                f"{'/'.join(want_dtype[kind])}")
            if tuple(loc.shape) != tuple(shape) or loc.nbytes != nbytes:
                raise PmoeError(f"{layout.path}: {name} of expert {e} is {loc.shape} "
                                f"({loc.nbytes} B), the slot expects {shape} ({nbytes} B)")


class _Files:
    """One read-only descriptor per checkpoint file."""

    def __init__(self):
        self.fds = {}

    def pread_into(self, loc: TensorLoc, out: np.ndarray) -> None:
        fd = self.fds.get(loc.file)
        if fd is None:
            fd = self.fds[loc.file] = os.open(loc.file, os.O_RDONLY)
        mv = memoryview(out).cast("B")
        done = 0
        while done < loc.nbytes:
            n = os.preadv(fd, [mv[done:]], loc.offset + done)
            if n <= 0:
                raise OSError(f"short read of {loc.file} at {loc.offset + done}")
            done += n

    def close(self):
        for fd in self.fds.values():
            os.close(fd)
        self.fds = {}


def read_expert(layout: ExpertLayout, e: int, g: Geom, out: np.ndarray, files=None) -> None:
    """Expert e's nine byte ranges into ``out`` (uint8, one slot:
    ``g.expert_bytes``) at the slot's component offsets."""
    if out.dtype != np.uint8 or out.size != int(g.expert_bytes):
        raise ValueError(f"out must be {int(g.expert_bytes)} uint8, got {out.size} {out.dtype}")
    own = files is None
    files = files or _Files()
    try:
        for c, name in enumerate(COMPONENTS):
            off, nb = int(g.off[c]), int(g.nbytes[c])
            loc = layout.loc(name, e)
            if loc.nbytes != nb:
                raise PmoeError(f"{layout.path}: {name} of expert {e} is {loc.nbytes} B, the "
                                f"slot holds {nb} B")
            files.pread_into(loc, out[off:off + nb])
    finally:
        if own:
            files.close()


def fill_host_store(store, layouts, g: Geom) -> None:
    """Every expert of ``layouts`` (one per store layer, in order) into the
    pinned host store (cache.HostExpertStore), after checking shapes."""
    if len(layouts) != store.n_layers:
        raise ValueError(f"{len(layouts)} layer layouts for a store of {store.n_layers} layers")
    files = _Files()
    try:
        for li, lay in enumerate(layouts):
            check_layout(lay, g)
            if lay.n_experts != store.n_experts:
                raise PmoeError(f"{lay.path}: {lay.n_experts} experts, the store holds "
                                f"{store.n_experts}")
            for e in range(lay.n_experts):
                read_expert(lay, e, g, store.expert_view(li, e), files)
    finally:
        files.close()
