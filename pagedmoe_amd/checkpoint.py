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

import json
import os
import re
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
    offset of its first element and its size (the record of
    safetensors_index.py:61-89)."""

    file: str
    dtype: str
    shape: tuple
    offset: int
    nbytes: int

    def row_bytes(self) -> int:
        """Bytes of one leading-index entry, from the trailing shape and the
        element size; the stacked tensor's size must be a whole multiple."""
        item = _ITEMSIZE.get(self.dtype)
        if item is None:
            raise PmoeError(f"{self.file}: dtype {self.dtype} has no fixed element size")
        per = item * int(np.prod(self.shape[1:], dtype=np.int64))
        if per * self.shape[0] != self.nbytes:
            raise PmoeError(f"{self.file}: {self.nbytes} B is not {self.shape[0]} entries of "
                            f"{per} B")
        return per

    def expert_slice(self, e: int) -> "TensorLoc":
        """Entry e of a stacked [E, ...] tensor (an expert's range)."""
        if not 0 <= e < self.shape[0]:
            raise IndexError(f"expert {e} outside a stack of {self.shape[0]}")
        per = self.row_bytes()
        return TensorLoc(self.file, self.dtype, tuple(self.shape[1:]), self.offset + per * e, per)


def shard_files(model_dir) -> list:
    """The checkpoint's safetensors shards: the files a
    ``model.safetensors.index.json`` weight map names when the directory has
    one, else every ``*.safetensors`` file in it, in name order."""
    root = Path(model_dir)
    index_file = root / "model.safetensors.index.json"
    if index_file.is_file():
        weight_map = json.loads(index_file.read_text()).get("weight_map", {})
        return [root / name for name in sorted(set(weight_map.values()))]
    return sorted(root.glob("*.safetensors"))


def _header(path: Path):
    """(absolute offset of the data section, {name: meta}) of one shard.

    A safetensors file starts with a u64 little-endian length n, then n bytes
    of JSON mapping each tensor to {dtype, shape, data_offsets} (offsets
    relative to the data section, which starts at 8 + n), plus an optional
    "__metadata__" entry."""
    fd = os.open(path, os.O_RDONLY)
    try:
        size = os.fstat(fd).st_size
        head = os.pread(fd, 8, 0)
        n = int.from_bytes(head, "little") if len(head) == 8 else -1
        if n < 2 or 8 + n > size:
            raise PmoeError(f"{path}: not a safetensors file ({size} B, header length {n})")
        meta = json.loads(os.pread(fd, n, 8))
    finally:
        os.close(fd)
    meta.pop("__metadata__", None)
    return 8 + n, meta, size


def read_headers(model_dir) -> dict:
    """Every tensor of the checkpoint's shards -> TensorLoc, from the file
    headers alone (no tensor data is read)."""
    files = shard_files(model_dir)
    if not files:
        raise FileNotFoundError(f"{model_dir}: no safetensors shards (no index file and no "
                                "*.safetensors)")
    index = {}
    for path in files:
        data, meta, size = _header(path)
        for name, m in meta.items():
            lo, hi = (int(v) for v in m["data_offsets"])
            if not 0 <= lo <= hi or data + hi > size:
                raise PmoeError(f"{path}: {name} spans [{lo}, {hi}) past the end of the file")
            loc = TensorLoc(str(path), m["dtype"], tuple(int(d) for d in m["shape"]), data + lo,
                            hi - lo)
            item = _ITEMSIZE.get(loc.dtype)
            if item and int(np.prod(loc.shape, dtype=np.int64)) * item != loc.nbytes:
                raise ValueError(f"{path}: {name} has {loc.nbytes} bytes for shape {loc.shape} "
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
