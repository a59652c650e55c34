"""Slot-addressed HBM storage for uniformly shaped quantized experts.

Counterpart of the reference's ``SlabStore`` (slab.py:82-183).  The reference
keeps one ``[slots, *expert_shape]`` array per component in unified memory
and preads into it.  Here a slab is ONE device allocation of
``slots * expert_bytes`` bytes laid out expert-major: slot s holds the nine
components of one expert back to back (``pmoe_geom.off``), so a miss is a
single contiguous host->HBM copy and every kernel addresses an expert as
``base + slot * expert_bytes``.  ``compute(name)`` still hands out the
reference's ``[slots, *shape]`` view of one component (a strided view, no
copy).
"""

from __future__ import annotations

import torch

from ._lib import COMPONENTS, Geom, geom as make_geom


def component_specs(g: Geom) -> dict:
    """name -> (per-expert shape, torch dtype, nbytes, offset)."""
    d, i, b = g.hidden, g.inter, g.bits
    gs = g.group
    shapes = {
        "gate_proj.weight": ((i, d * b // 32), torch.int32),
        "gate_proj.scales": ((i, d // gs), torch.bfloat16),
        "gate_proj.biases": ((i, d // gs), torch.bfloat16),
        "up_proj.weight": ((i, d * b // 32), torch.int32),
        "up_proj.scales": ((i, d // gs), torch.bfloat16),
        "up_proj.biases": ((i, d // gs), torch.bfloat16),
        "down_proj.weight": ((d, i * b // 32), torch.int32),
        "down_proj.scales": ((d, i // gs), torch.bfloat16),
        "down_proj.biases": ((d, i // gs), torch.bfloat16),
    }
    out = {}
    for c, name in enumerate(COMPONENTS):
        shape, dt = shapes[name]
        out[name] = (shape, dt, int(g.nbytes[c]), int(g.off[c]))
    return out


class SlabStore:
    """``slots`` expert slots of geometry ``g`` in one HBM allocation."""

    def __init__(self, g: Geom, slots: int, device="cuda", zero: bool = True):
        if slots < 1:
            raise ValueError(f"slab needs at least one slot, got {slots}")
        self.geom = g
        self.slots = int(slots)
        self.expert_bytes = int(g.expert_bytes)
        self.specs = component_specs(g)
        self.names = tuple(COMPONENTS)
        alloc = torch.zeros if zero else torch.empty
        self.buf = alloc(self.slots * self.expert_bytes, dtype=torch.uint8, device=device)
        self.nbytes = self.buf.numel()

    @classmethod
    def for_shape(cls, hidden: int, inter: int, bits: int, slots: int, device="cuda"):
        return cls(make_geom(hidden, inter, bits), slots, device)

    @property
    def data_ptr(self) -> int:
        return self.buf.data_ptr()

    def release(self) -> None:
        """Drop the allocation (callers must hold no views)."""
        self.buf = None
        self.nbytes = 0

    def has(self, name: str) -> bool:
        return self.buf is not None and name in self.specs

    def slot_bytes(self, slot: int) -> torch.Tensor:
        """All bytes of one slot (uint8 [expert_bytes])."""
        return self.buf[slot * self.expert_bytes:(slot + 1) * self.expert_bytes]

    def dest(self, name: str, slot: int) -> torch.Tensor:
        """Writable byte range of one component of one slot."""
        shape, dt, nbytes, off = self.specs[name]
        base = slot * self.expert_bytes + off
        return self.buf[base:base + nbytes]

    def compute(self, name: str) -> torch.Tensor:
        """``[slots, *shape]`` strided view of one component."""
        shape, dt, nbytes, off = self.specs[name]
        item = torch.empty((), dtype=dt).element_size()
        flat = self.buf.view(dt)
        stride_slot = self.expert_bytes // item
        rm = []
        acc = 1
        for s in reversed(shape):
            rm.append(acc)
            acc *= s
        rm = list(reversed(rm))
        return flat.as_strided((self.slots, *shape), (stride_slot, *rm), off // item)

    def expert(self, name: str, slot: int) -> torch.Tensor:
        """One component of one slot, as ``shape``."""
        return self.compute(name)[slot]

    def write_expert(self, slot: int, comps: dict) -> None:
        """Copy one expert's components (device or host tensors with the
        component's shape/dtype, or raw bytes-compatible arrays) into slot."""
        for name in self.names:
            shape, dt, nbytes, off = self.specs[name]
            src = comps[name]
            if not isinstance(src, torch.Tensor):
                import numpy as np
                arr = np.ascontiguousarray(src)
                arr = arr.view(np.int32 if dt == torch.int32 else np.int16)
                src = torch.from_numpy(arr)
            src = src.reshape(shape)
            if src.dtype != dt:
                src = src.view(dt)
            self.expert(name, slot).copy_(src, non_blocking=False)

    def quantize_into(self, slot: int, proj: str, w: torch.Tensor) -> None:
        """Quantize fp32 weights w ([out, in] of projection `proj`) straight
        into slot's components (no staging copy)."""
        from . import kernels
        kernels.quantize(w, self.geom.bits, self.geom.group,
                         out=(self.expert(proj + ".weight", slot),
                              self.expert(proj + ".scales", slot),
                              self.expert(proj + ".biases", slot)))
