"""Shared helpers for the parity tests (tolerance checks, slab filling)."""

from __future__ import annotations

import numpy as np

from oracle import pmoe_oracle as O

# Layer-output tolerance against the float64 oracle: max-abs error within
# 1e-2 of the largest reference magnitude, relative L2 within 1e-2, and
# elementwise within 8 bf16 ulps of the reference plus 4e-3 of the reference
# scale.  The kernels round the SwiGLU intermediate h to bf16 (as mlx's
# gather_qmm outputs are bf16), which alone gives ~2.3e-3 relative L2 error;
# the 4e-3 floor is ~16 standard deviations of that noise.
RTOL = 1e-2


def check_close(got, ref, what="", rtol=RTOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(got - ref)
    assert err.max() <= rtol * scale, f"{what}: max err {err.max():.3e} vs scale {scale:.3e}"
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel <= rtol, f"{what}: rel L2 {rel:.3e}"
    ulp = np.abs(ref) * 2.0 ** -7
    bound = 8 * ulp + 4e-3 * scale
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(
            f"{what}: elementwise bound exceeded at {i}: got {got[i]:.6e} ref {ref[i]:.6e} "
            f"err {err[i]:.3e} bound {bound[i]:.3e}; {bad.sum()} of {bad.size} elements; "
            f"max err {err.max():.3e} scale {scale:.3e} relL2 {rel:.3e}")


def bf16_tensor_bits(t) -> np.ndarray:
    """bf16 torch tensor -> uint16 numpy bits."""
    import torch
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def bits_to_bf16_tensor(bits, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def expert_to_comps(ex: "O.Expert") -> dict:
    return {
        "gate_proj.weight": ex.gate.weight, "gate_proj.scales": ex.gate.scales,
        "gate_proj.biases": ex.gate.biases,
        "up_proj.weight": ex.up.weight, "up_proj.scales": ex.up.scales,
        "up_proj.biases": ex.up.biases,
        "down_proj.weight": ex.down.weight, "down_proj.scales": ex.down.scales,
        "down_proj.biases": ex.down.biases,
    }


def slot_to_expert(slab, slot) -> "O.Expert":
    """Read one slab slot back as an oracle Expert (packed bits, host)."""
    import torch
    g = slab.geom

    def qt(prefix, cols):
        w = slab.expert(prefix + ".weight", slot).cpu().numpy().view(np.uint32)
        s = slab.expert(prefix + ".scales", slot).cpu().view(torch.int16).numpy().view(np.uint16)
        b = slab.expert(prefix + ".biases", slot).cpu().view(torch.int16).numpy().view(np.uint16)
        return O.QTensor(w, s, b, g.bits, g.group, cols)

    return O.Expert(qt("gate_proj", g.hidden), qt("up_proj", g.hidden), qt("down_proj", g.inter))


def fill_slab_gpu(slab, slots, seed=0, std=0.02):
    """Random N(0, std) experts quantized on the GPU into the given slots."""
    import torch
    g = slab.geom
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    for slot in slots:
        for prefix, rows, cols in (("gate_proj", g.inter, g.hidden), ("up_proj", g.inter, g.hidden),
                                   ("down_proj", g.hidden, g.inter)):
            w = torch.randn((rows, cols), generator=gen, device="cuda", dtype=torch.float32) * std
            slab.quantize_into(slot, prefix, w)
