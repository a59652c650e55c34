"""Expert byte ranges of safetensors checkpoints (pagedmoe_amd/checkpoint.py),
the counterpart of the reference's safetensors_index.py:61-159 and
_layer_layout (streaming.py:2529-2572).  CPU only: synthetic checkpoints in
both on-disk layouts (stacked ``switch_mlp`` tensors and per-expert
``experts.<e>`` tensors) are written with safetensors' own writer, and every
byte read into slot layout is checked against the tensors it came from."""

import numpy as np
import pytest
import torch

from oracle import pmoe_oracle as O
from pagedmoe_amd import checkpoint as ck
from pagedmoe_amd._lib import COMPONENTS, PmoeError, geom

safetensors_torch = pytest.importorskip("safetensors.torch")

D, I, E = 512, 256, 6


def _experts(bits, seed):
    """E experts quantized by the oracle: name -> [E, ...] numpy arrays
    (weights u32, scales/biases bf16 bits)."""
    rng = np.random.default_rng(seed)
    out = {f"{p}.{c}": [] for p in ("gate_proj", "up_proj", "down_proj")
           for c in ("weight", "scales", "biases")}
    for _ in range(E):
        for p, (rows, cols) in (("gate_proj", (I, D)), ("up_proj", (I, D)), ("down_proj", (D, I))):
            qt = O.quantize(rng.standard_normal((rows, cols), dtype=np.float32) * 0.02, bits)
            out[f"{p}.weight"].append(qt.weight)
            out[f"{p}.scales"].append(qt.scales)
            out[f"{p}.biases"].append(qt.biases)
    return {k: np.stack(v) for k, v in out.items()}


def _tensor(name, a):
    if name.endswith("weight"):
        return torch.from_numpy(a.astype(np.uint32).view(np.int32)).contiguous()
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).contiguous()


def _write_stacked(path, layers, prefix="model"):
    tensors = {}
    for n, comps in layers.items():
        for name, a in comps.items():
            tensors[f"{prefix}.layers.{n}.mlp.switch_mlp.{name}"] = _tensor(name, a)
    tensors[f"{prefix}.embed_tokens.weight"] = torch.zeros(4, 8, dtype=torch.bfloat16)
    safetensors_torch.save_file(tensors, str(path))


def _write_per_expert(path, layers):
    tensors = {}
    for n, comps in layers.items():
        for name, a in comps.items():
            proj, comp = name.split(".")
            for e in range(a.shape[0]):
                tensors[f"model.layers.{n}.mlp.experts.{e}.{proj}.{comp}"] = _tensor(name, a[e])
    safetensors_torch.save_file(tensors, str(path))


def _slot_expected(g, comps, e):
    out = np.zeros(int(g.expert_bytes), np.uint8)
    for c, name in enumerate(COMPONENTS):
        raw = np.ascontiguousarray(comps[name][e]).view(np.uint8).reshape(-1)
        out[int(g.off[c]):int(g.off[c]) + raw.size] = raw
    return out


@pytest.mark.parametrize("bits", [4, 6])
def test_stacked_layout_reads_each_expert_into_slot_layout(tmp_path, bits):
    layers = {1: _experts(bits, 1), 3: _experts(bits, 3)}
    _write_stacked(tmp_path / "model-00001-of-00001.safetensors", layers)
    index = ck.read_headers(tmp_path)
    # header offsets agree with safetensors' own reader
    ref = safetensors_torch.load_file(str(tmp_path / "model-00001-of-00001.safetensors"))
    for name, loc in index.items():
        with open(loc.file, "rb") as f:
            f.seek(loc.offset)
            raw = f.read(loc.nbytes)
        assert raw == ref[name].contiguous().view(torch.uint8).numpy().tobytes(), name
    found = ck.find_moe_layers(index)
    assert found == [(1, "model.layers.1.mlp.switch_mlp"), (3, "model.layers.3.mlp.switch_mlp")]
    lay = ck.layer_layout(found[1][1], index)
    assert lay.stacked and lay.n_experts == E
    assert lay.geometry() == (D, I, bits)
    g = geom(D, I, bits)
    ck.check_layout(lay, g)
    for e in range(E):
        slot = np.zeros(int(g.expert_bytes), np.uint8)
        ck.read_expert(lay, e, g, slot)
        assert np.array_equal(slot, _slot_expected(g, layers[3], e)), f"expert {e}"
        # the slot's weight words dequantize to the source projection
        c = COMPONENTS.index("down_proj.weight")
        w = slot[int(g.off[c]):int(g.off[c]) + int(g.nbytes[c])].view(np.uint32).reshape(D, -1)
        s = slot[int(g.off[c + 1]):int(g.off[c + 1]) + int(g.nbytes[c + 1])].view(np.uint16)
        b = slot[int(g.off[c + 2]):int(g.off[c + 2]) + int(g.nbytes[c + 2])].view(np.uint16)
        got = O.dequant_f32(O.QTensor(w, s.reshape(D, -1), b.reshape(D, -1), bits, 64, I))
        src = layers[3]
        want = O.dequant_f32(O.QTensor(src["down_proj.weight"][e], src["down_proj.scales"][e],
                                       src["down_proj.biases"][e], bits, 64, I))
        assert np.array_equal(got, want)


def test_per_expert_layout_gives_the_same_slots(tmp_path):
    comps = _experts(4, 7)
    (tmp_path / "a").mkdir()
    (tmp_path / "b").mkdir()
    _write_stacked(tmp_path / "a" / "model.safetensors", {0: comps})
    _write_per_expert(tmp_path / "b" / "model.safetensors", {0: comps})
    g = geom(D, I, 4)
    la = ck.layer_layout("model.layers.0.mlp.switch_mlp", ck.read_headers(tmp_path / "a"))
    ib = ck.read_headers(tmp_path / "b")
    assert ck.find_moe_layers(ib) == [(0, "model.layers.0.mlp.switch_mlp")]
    lb = ck.layer_layout("model.layers.0.mlp.switch_mlp", ib)
    assert not lb.stacked and lb.n_experts == E
    for e in range(E):
        sa = np.zeros(int(g.expert_bytes), np.uint8)
        sb = np.zeros(int(g.expert_bytes), np.uint8)
        ck.read_expert(la, e, g, sa)
        ck.read_expert(lb, e, g, sb)
        assert np.array_equal(sa, sb)
        assert np.array_equal(sa, _slot_expected(g, comps, e))


def test_prefixed_names_and_sharded_files(tmp_path):
    # experts of two layers in two files, under a language_model. prefix
    _write_stacked(tmp_path / "model-00001-of-00002.safetensors", {0: _experts(4, 11)},
                   prefix="language_model.model")
    _write_stacked(tmp_path / "model-00002-of-00002.safetensors", {5: _experts(4, 12)},
                   prefix="language_model.model")
    index = ck.read_headers(tmp_path)
    assert [n for n, _ in ck.find_moe_layers(index)] == [0, 5]
    lay = ck.layer_layout("language_model.model.layers.5.mlp.switch_mlp", index)
    assert lay.loc("gate_proj.weight", 0).file.endswith("00002-of-00002.safetensors")


def test_mismatched_checkpoints_are_refused(tmp_path):
    comps = _experts(4, 5)
    # scales stored as F16 instead of bf16
    bad = dict(comps)
    tensors = {f"model.layers.0.mlp.switch_mlp.{k}": _tensor(k, v) for k, v in bad.items()}
    tensors["model.layers.0.mlp.switch_mlp.up_proj.scales"] = torch.zeros(
        E, I, D // 64, dtype=torch.float16)
    safetensors_torch.save_file(tensors, str(tmp_path / "model.safetensors"))
    lay = ck.layer_layout("model.layers.0.mlp.switch_mlp", ck.read_headers(tmp_path))
    with pytest.raises(PmoeError, match="up_proj.scales is F16"):
        ck.check_layout(lay, geom(D, I, 4))
    # a slot geometry that does not match the checkpoint
    good = tmp_path / "good"
    good.mkdir()
    _write_stacked(good / "model.safetensors", {0: comps})
    lay = ck.layer_layout("model.layers.0.mlp.switch_mlp", ck.read_headers(good))
    with pytest.raises(PmoeError, match="slot expects"):
        ck.check_layout(lay, geom(D, 2 * I, 4))
    # a dense (unquantized) MLP has no expert tensors
    dense = tmp_path / "dense"
    dense.mkdir()
    safetensors_torch.save_file({"model.layers.0.mlp.gate_proj.weight": torch.zeros(4, 4)},
                                str(dense / "model.safetensors"))
    assert ck.find_moe_layers(ck.read_headers(dense)) == []
    with pytest.raises(KeyError):
        ck.layer_layout("model.layers.0.mlp.switch_mlp", ck.read_headers(dense))
    with pytest.raises(FileNotFoundError):
        ck.read_headers(tmp_path / "nowhere")
