#!/usr/bin/env python3
"""MoE-layer throughput of the routed-expert hot path on one MI355X.

One step = one MoE layer (router -> top-k -> dispatch -> quantized SwiGLU
experts -> combine) over one batch of tokens.  Default workload: the
Qwen3-235B-A22B-shaped decode layer (hidden 4096, 128 experts,
moe_intermediate 1536, top-8 softmax+renorm, 4-bit affine g64, bf16 scales and
biases, all experts resident in the HBM slab), batch 1 (batch 8 reported in
"extra").  Weights are synthetic: N(0, 0.02) quantized on the GPU; activations
N(0, 1) bf16; every step routes a fresh token.  Steps cycle over `--layers`
distinct layers (default 8, ~11 GB of experts) so no step finds the previous
step's experts in the 256 MB last-level cache.

The timed loop replays a HIP graph of G consecutive layer steps, G the
largest divisor of `--steps` up to 64, `--steps`/G times, so exactly
`--steps` steps are timed (launch overhead excluded, as in the reference's
one-graph-per-token decode); inputs are resident in HBM before timing starts,
and HIP events on the replay stream bracket the timed replays.  Before that,
untimed: `--warmup` eager steps, one eager pass of G steps with every kernel
bracketed by HIP events (per-kernel durations), one pass of G steps to warm
the capture stream and one warm replay; "warmup" in the JSON line counts all
of them.  roofline.achieved = algorithmic expert-weight bytes per launch /
the dominant kernel's average duration: for the one-launch decode layer (the
batch-1 default) a step is that one launch, so its duration is the
event-timed graph step; for the three-launch decode it is the kernel's
event-timed eager average.  roofline.traffic comes from the rocprofv3
FETCH_SIZE + WRITE_SIZE profile committed under profiles/, scaled by the
probe kernels' counters, and only when that profile's source hash matches
the kernel sources being run.

Prints ONE JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

WORKLOADS = {
    "qwen3-235b-decode": dict(hidden=4096, experts=128, inter=1536, top_k=8, bits=4,
                              scoring="softmax"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_layers(g, spec, n_layers, device, seed=0):
    """Slab with n_layers * E slots (slot = layer*E + e), router weights and
    the per-layer expert->slot tables."""
    import torch

    from pagedmoe_amd.slab import SlabStore

    E, D, I = spec["experts"], spec["hidden"], spec["inter"]
    slab = SlabStore(g, n_layers * E, device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for slot in range(n_layers * E):
        for prefix, rows, cols in (("gate_proj", I, D), ("up_proj", I, D), ("down_proj", D, I)):
            w = torch.randn((rows, cols), generator=gen, device=device) * 0.02
            slab.quantize_into(slot, prefix, w)
    gate = (torch.randn((n_layers, E, D), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    tables = (torch.arange(n_layers, device=device, dtype=torch.int32)[:, None] * E
              + torch.arange(E, device=device, dtype=torch.int32)[None, :]).contiguous()
    return slab, gate, tables


# kernel -> the sources its code comes from (the traffic profile is valid
# only for the build of these files it was measured on; the Makefile holds
# per-file compiler flags)
KERNEL_SOURCES = {
    "decode_fused_kernel": ["decode_fused.hip", "gemv_common.h", "route_common.h",
                            "pmoe_internal.h", "pmoe_kernels.h", "Makefile"],
    "decode_xcd_kernel": ["decode_fused.hip", "gemv_common.h", "route_common.h",
                          "pmoe_internal.h", "pmoe_kernels.h", "Makefile"],
    "gateup_routed_kernel": ["decode.hip", "gemv_common.h", "route_common.h",
                             "pmoe_internal.h", "pmoe_kernels.h"],
    "prefill": ["prefill.hip", "dispatch.hip", "moe.hip", "pmoe_internal.h", "pmoe_kernels.h"],
}


def source_hash(kernel: str) -> str:
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES[kernel]:
        h.update(name.encode())
        h.update((ROOT / "pagedmoe_amd" / "csrc" / name).read_bytes())
    return h.hexdigest()[:16]


def load_traffic(name: str, kernel: str):
    """(bytes per launch, note) from profiles/traffic_<name>.json when its
    source hash matches the current sources of `kernel`."""
    f = ROOT / "profiles" / f"traffic_{name}.json"
    if not f.exists():
        return None, f"no profiles/{f.name}"
    try:
        tf = json.loads(f.read_text())
    except (ValueError, OSError) as e:
        return None, f"profiles/{f.name}: {e}"
    if tf.get("kernel") != kernel:
        return None, f"profiles/{f.name} is for {tf.get('kernel')}, not {kernel}"
    if tf.get("source_hash") != source_hash(kernel):
        return None, (f"profiles/{f.name} was measured on other sources "
                      f"({tf.get('source_hash')} vs {source_hash(kernel)})")
    return tf.get("bytes_per_launch"), f"profiles/{f.name} (source {tf['source_hash']})"


def graph_len(steps: int, cap: int = 64) -> int:
    """Largest divisor of steps that is at most cap: the graph length that
    lets whole replays time exactly `steps` steps."""
    for n in range(min(cap, steps), 0, -1):
        if steps % n == 0:
            return n
    return 1


def run_decode(args, g, spec, slab, gate, tables, batch, device):
    import torch

    from pagedmoe_amd import kernels as K
    from pagedmoe_amd._lib import KernelTimer

    E, D, k = spec["experts"], spec["hidden"], spec["top_k"]
    L = args.layers
    seq = graph_len(args.steps)                   # layer steps per graph
    rc = K.route_cfg(spec["scoring"], E, k)
    gen = torch.Generator(device=device)
    gen.manual_seed(1000 + batch)
    x = torch.randn((seq, batch, D), generator=gen, device=device).to(torch.bfloat16)
    out = torch.empty((seq, batch, D), dtype=torch.bfloat16, device=device)
    inds = torch.empty((seq, batch, k), dtype=torch.int32, device=device)
    wts = torch.empty((seq, batch, k), dtype=torch.float32, device=device)
    ws = K.moe_workspace(g, batch, k, 0, E, device, fresh=True)  # private to the graph

    def step(i):
        layer = i % L
        K.moe_block(g, rc, slab.buf, tables[layer], gate[layer], x[i], out=out[i],
                    inds=inds[i], weights=wts[i], ws=ws)

    def run_seq():
        for i in range(seq):
            step(i)

    # eager warmup (also validates the call path): exactly --warmup steps
    for i in range(args.warmup):
        step(i % seq)
    torch.cuda.synchronize()

    # per-kernel durations: one eager pass with event brackets
    with KernelTimer() as kt:
        run_seq()
    torch.cuda.synchronize()

    # graph of `seq` layer steps
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_seq()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run_seq()
    graph.replay()
    torch.cuda.synchronize()
    reps = args.steps // seq
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()  # the replays run on this (the current) stream
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    steps_timed = reps * seq
    ms = (t1 - t0) * 1e3 / steps_timed
    gpu_ms = ev0.elapsed_time(ev1) / steps_timed

    # eager wall time for transparency
    torch.cuda.synchronize()
    e0 = time.perf_counter()
    run_seq()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - e0) * 1e3 / seq

    # algorithmic bytes: distinct experts per step x per-expert bytes
    ids = inds.cpu().numpy().reshape(seq, -1)
    uniq = [len(set(r.tolist())) for r in ids]
    mean_unique = sum(uniq) / len(uniq)
    gateup_bytes = int(g.nbytes[0] + g.nbytes[1] + g.nbytes[2]) * 2
    down_bytes = int(g.nbytes[6] + g.nbytes[7] + g.nbytes[8])
    layer_bytes = mean_unique * (gateup_bytes + down_bytes)
    res = {
        "batch": batch,
        "ms_per_step": ms,
        "gpu_ms_per_step": gpu_ms,
        "tokens_per_s": batch / (ms / 1e3),
        "steps_timed": steps_timed,
        "graph_steps": seq,
        "graph_replays_timed": reps,
        "untimed_steps": args.warmup + 3 * seq,
        "eager_ms_per_step": eager_ms,
        "mean_unique_experts": mean_unique,
        "expert_bytes_per_step": mean_unique * int(g.expert_bytes),
        "kernels": {},
    }
    for name, (tot, cnt) in kt.result.items():
        res["kernels"][name] = {"avg_us": tot * 1e3 / cnt, "launches": cnt}
    # kernel launches in the timer pass = reps_timer * seq; each processed the
    # distinct experts of its step
    step_bytes_gu = mean_unique * gateup_bytes
    step_bytes_dn = mean_unique * down_bytes
    ku = res["kernels"].get("qgemv_gateup")
    kd = res["kernels"].get("qgemv_down")
    if ku:
        res["gateup_gbs"] = step_bytes_gu / (ku["avg_us"] * 1e-6) / 1e9
    if kd:
        res["down_gbs"] = step_bytes_dn / (kd["avg_us"] * 1e-6) / 1e9
    kf = res["kernels"].get("decode_fused") or res["kernels"].get("decode_xcd")
    if kf:
        # a fused step is this one launch: its duration in the timed region
        # is the event-timed graph step (launch gaps included)
        kf["graph_avg_us"] = gpu_ms * 1e3
        res["fused_gbs"] = layer_bytes / (gpu_ms * 1e-3) / 1e9
    res["_layer_bytes"] = layer_bytes
    res["layer_expert_gbs"] = res["expert_bytes_per_step"] / (ms * 1e-3) / 1e9
    res["_gateup_step_bytes"] = step_bytes_gu
    if ws is not None:
        res["workspace_error"] = K.workspace_error(ws)
    return res


def run_prefill(args, g, spec, slab, gate, tables, device, tokens=2048):
    """The same layers at a `tokens`-token prefill chunk: router logits
    skewed by a per-expert N(0,1) bias (uneven expert loads), expert-sorted
    dispatch feeding the dequant -> bf16 MFMA GEMMs.  Timed as HIP-graph
    replays of one layer step per layer; per-kernel averages from an
    event-bracketed eager pass."""
    import torch

    from pagedmoe_amd import kernels as K
    from pagedmoe_amd._lib import KernelTimer

    E, D, I, k = spec["experts"], spec["hidden"], spec["inter"], spec["top_k"]
    L = args.layers
    rc = K.route_cfg(spec["scoring"], E, k)
    gen = torch.Generator(device=device)
    gen.manual_seed(3000)
    x = torch.randn((L, tokens, D), generator=gen, device=device).to(torch.bfloat16)
    lb = torch.randn((L, E), generator=gen, device=device)
    out = torch.empty((L, tokens, D), dtype=torch.bfloat16, device=device)
    inds = torch.empty((L, tokens, k), dtype=torch.int32, device=device)
    wts = torch.empty((L, tokens, k), dtype=torch.float32, device=device)
    ws = K.moe_workspace(g, tokens, k, 0, E, device, fresh=True)

    def run_seq():
        for i in range(L):
            K.moe_block(g, rc, slab.buf, tables[i], gate[i], x[i], logit_bias=lb[i], out=out[i],
                        inds=inds[i], weights=wts[i], ws=ws)

    run_seq()
    torch.cuda.synchronize()
    with KernelTimer() as kt:
        run_seq()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_seq()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run_seq()
    graph.replay()
    torch.cuda.synchronize()
    reps = max(2, args.prefill_reps)
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / (reps * L)
    rows = tokens * k
    flops_gu = 4.0 * D * I * rows
    flops_dn = 2.0 * D * I * rows
    res = {"tokens": tokens, "ms_per_step": ms, "tokens_per_s": tokens / (ms * 1e-3),
           "expert_tflops": (flops_gu + flops_dn) / (ms * 1e-3) / 1e12,
           "mfma_frac_layer": (flops_gu + flops_dn) / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
           "expert_flops_per_step": flops_gu + flops_dn,
           "router_flops_per_step": 2.0 * tokens * D * E,
           "max_expert_rows": int(torch.bincount(inds[0].reshape(-1).long(), minlength=E).max()),
           "kernels": {}}
    for name, (tot, cnt) in kt.result.items():
        res["kernels"][name] = {"avg_us": tot * 1e3 / cnt, "launches": cnt}
    for name, fl in (("prefill_gateup", flops_gu), ("prefill_down", flops_dn)):
        kr = res["kernels"].get(name)
        if kr:
            kr["tflops"] = fl / (kr["avg_us"] * 1e-6) / 1e12
            kr["mfma_frac"] = kr["tflops"] / MFMA_BF16_PEAK_TFLOPS
    return res


def run_paging(args, device, tokens=256, warm=96):
    """DeepSeek-V3/Kimi-K2-shaped layer decode with paging: hidden 7168, 384
    routed experts + 1 shared, moe_intermediate 2048, 4-bit g64, batch 1.
    The HBM slab holds 96 routed slots (+ the shared expert's pinned slot);
    every expert lives in a pinned host store and misses are copied in by the
    copy engine (side streams, event hand-off).  Expert ids follow a seeded
    Zipf(1.1) popularity (ranks through a fixed permutation; 8 distinct ids
    per token, sigmoid-style weights summing to 2.5).  Reports tokens/s, hit
    rate, H2D bytes and rate, and the stall (wall time not spent in kernels)."""
    import numpy as np
    import torch

    from pagedmoe_amd import kernels as K
    from pagedmoe_amd._lib import KernelTimer, geom
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore
    from pagedmoe_amd.slab import SlabStore

    D, E, I, k, slots = 7168, 384, 2048, 8, 96
    g = geom(D, I, 4)
    t0 = time.perf_counter()
    store = HostExpertStore(g, 1, E)
    tmp = SlabStore(g, 1, device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(4)

    def synth(slab, slot):
        for prefix, rows, cols in (("gate_proj", I, D), ("up_proj", I, D), ("down_proj", D, I)):
            slab.quantize_into(slot, prefix, torch.randn((rows, cols), generator=gen,
                                                         device=device) * 0.02)

    for e in range(E):
        synth(tmp, 0)
        store.write_from_slot(0, e, tmp, 0)
    tmp.release()
    cache = ExpertCache(g, slots, [0], E, host_store=store, n_shared=1, device=device)
    synth(cache.slab, cache.shared_slot(0))
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0

    rng = np.random.default_rng(0)
    perm = rng.permutation(E)
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    pop = pop / pop.sum()
    n_tok = warm + tokens
    ids = np.stack([perm[rng.choice(E, k, replace=False, p=pop)] for _ in range(n_tok)])
    w = rng.random((n_tok, k)).astype(np.float32) + 0.1
    w = w / w.sum(1, keepdims=True) * 2.5
    inds = torch.from_numpy(ids.astype(np.int32)).to(device)
    wts = torch.from_numpy(w).to(device)
    x = torch.randn((n_tok, 1, D), generator=gen, device=device).to(torch.bfloat16)
    out = torch.empty((n_tok, 1, D), dtype=torch.bfloat16, device=device)
    table = cache.table_ptr(0)
    shared = cache.shared_slot(0)

    def step(i):
        cache.fetch(0, ids[i].tolist())
        out[i] = K.moe_experts(g, cache.slab.buf, table, E, x[i], inds[i:i + 1],
                               wts[i:i + 1], shared_slot=shared)

    for i in range(warm):
        step(i)
    torch.cuda.synchronize()
    st0 = cache.stats()
    with KernelTimer() as kt:
        c0 = time.perf_counter()
        for i in range(warm, n_tok):
            step(i)
        torch.cuda.synchronize()
        wall = time.perf_counter() - c0
    st1 = cache.stats()
    hits = st1["hits"] - st0["hits"]
    misses = st1["misses"] - st0["misses"]
    h2d = (st1["h2d_gb"] - st0["h2d_gb"]) * 1e9
    kern_s = sum(tot for tot, _ in kt.result.values()) / 1e3
    stall = max(0.0, wall - kern_s)
    expert_bytes = int(g.expert_bytes)
    res = {
        "workload": "DeepSeek-V3/Kimi-K2-shaped layer decode with paging",
        "hidden": D, "experts": E, "shared_experts": 1, "moe_intermediate": I, "top_k": k,
        "bits": 4, "slab_slots": slots, "popularity": "Zipf(1.1), seed 0", "batch": 1,
        "tokens_timed": tokens, "warmup_tokens": warm,
        "tokens_per_s": tokens / wall, "ms_per_token": wall * 1e3 / tokens,
        "hit_rate": hits / max(1, hits + misses), "misses_per_token": misses / tokens,
        "h2d_gb": h2d / 1e9, "h2d_gbs": h2d / stall / 1e9 if stall > 0 else None,
        "stall_ms_per_token": stall * 1e3 / tokens,
        "kernel_ms_per_token": kern_s * 1e3 / tokens,
        "hbm_expert_bytes_per_token": (k + 1) * expert_bytes,
        "kernel_hbm_gbs": (k + 1) * expert_bytes * tokens / kern_s / 1e9 if kern_s else None,
        "setup_s": setup_s,
        "note": "stall = wall time - sum of kernel times (the compute stream waiting on host "
                "copies); h2d_gbs = copied bytes / stall; no speculative prefetch",
    }
    cache.close()
    store.close()
    return res


def run_paging_predicted(args, device, n_layers=5, tokens=96, warm=32, auto_tokens=480,
                         slots_per_layer=96, alpha=0.25):
    """The DeepSeek-V3/Kimi-K2-shaped layers paged through a slab of 96
    routed slots per layer, decoded through SigmoidGroupMoEBlocks (router,
    sigmoid + correction bias, 8 groups / top-4 / top-8, scale 2.5, shared
    expert), with and without route prediction.  Synthetic residual stream:
    each layer's input is the previous one's plus alpha * N(0, 1), and a
    per-expert logit bias of -1.1 * log(rank) (ranks through a fixed
    permutation) skews popularity toward a Zipf(1.1)-like profile.  Both runs
    see the same tokens and share one pinned host store; reports per mode
    tokens/s, stall per token, hit rate, misses per token, and for prediction
    the precision and the speculative reads started and claimed; a third run
    leaves the choice to the A/B governor (predict mode "auto") over
    auto_tokens tokens and reports what it decided."""
    import numpy as np
    import torch

    from pagedmoe_amd import config as CF
    from pagedmoe_amd._lib import KernelTimer, geom
    from pagedmoe_amd.cache import ExpertCache, HostExpertStore
    from pagedmoe_amd.slab import SlabStore
    from pagedmoe_amd.streaming import SigmoidGroupMoEBlock, StreamedSwitchGLU, patch_model

    D, E, I, k = 7168, 384, 2048, 8
    g = geom(D, I, 4)
    t0 = time.perf_counter()
    store = HostExpertStore(g, n_layers, E)
    tmp = SlabStore(g, 1, device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(44)

    def synth(slab, slot):
        for prefix, rows, cols in (("gate_proj", I, D), ("up_proj", I, D), ("down_proj", D, I)):
            slab.quantize_into(slot, prefix, torch.randn((rows, cols), generator=gen,
                                                         device=device) * 0.02)

    for e in range(E):                 # one set of synthetic experts, every layer a copy
        synth(tmp, 0)
        store.write_from_slot(0, e, tmp, 0)
    one = store.bytes[:E * store.expert_bytes]
    for li in range(1, n_layers):
        store.bytes[li * E * store.expert_bytes:(li + 1) * E * store.expert_bytes] = one
    rng = np.random.default_rng(45)
    gates = [(torch.randn((E, D), generator=gen, device=device) * 0.02).to(torch.bfloat16)
             for _ in range(n_layers)]
    corr = [torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32)).to(device)
            for _ in range(n_layers)]
    skew = []
    for _ in range(n_layers):
        rank = np.empty(E)
        rank[rng.permutation(E)] = np.arange(1, E + 1)
        skew.append(torch.from_numpy((-1.1 * np.log(rank)).astype(np.float32)).to(device))
    setup_s = time.perf_counter() - t0

    class Layer(torch.nn.Module):
        def __init__(self, mlp):
            super().__init__()
            self.mlp = mlp

    def build(mode):
        keys = [f"layers.{li}.mlp.switch_mlp" for li in range(n_layers)]
        cache = ExpertCache(g, slots_per_layer * n_layers, keys, E, host_store=store,
                            n_shared=1, device=device, stage_slots=0)
        for li in range(n_layers):
            cache.slab.slot_bytes(cache.shared_slot(keys[li])).copy_(tmp_shared)
        model = torch.nn.Module()
        blocks = []
        for li in range(n_layers):
            st = StreamedSwitchGLU(keys[li], None, cache)
            blk = SigmoidGroupMoEBlock(gates[li], corr[li], st, top_k=k, n_group=8, topk_group=4,
                                       routed_scaling_factor=2.5)
            blk.logit_bias = skew[li]
            blocks.append(blk)
        model.layers = torch.nn.ModuleList([Layer(b) for b in blocks])
        # patch_model's ring over the streamed seams already in place
        from pagedmoe_amd.ring import PrefetchRing
        ring = PrefetchRing([b.switch_mlp for b in blocks], cache)
        for b in blocks:
            b.switch_mlp.pred = b
        ring.governor.set_mode(mode)
        return model, cache, ring

    tmp_shared = torch.empty(int(g.expert_bytes), dtype=torch.uint8, device=device)
    synth(tmp, 0)
    tmp_shared.copy_(tmp.slot_bytes(0))
    tmp.release()
    del patch_model
    out = {"config": {"workload": "DeepSeek-V3/Kimi-K2-shaped paged decode, route prediction",
                      "layers": n_layers, "hidden": D, "experts": E, "shared_experts": 1,
                      "moe_intermediate": I, "top_k": k, "bits": 4,
                      "slab_slots": slots_per_layer * n_layers,
                      "residual_update": f"x_(l+1) = x_l + {alpha} * N(0,1)",
                      "popularity": "logit bias -1.1*log(rank), ranks permuted (seed 45)",
                      "predict_depth": CF.PREDICT_DEPTH, "predict_slack": CF.PREDICT_SLACK,
                      "tokens_timed": tokens, "warmup_tokens": warm, "setup_s": setup_s}}
    for name, mode in (("no_prediction", "off"), ("prediction", "on"), ("governor", "auto")):
        model, cache, ring = build(mode)
        n_tok = auto_tokens if mode == "auto" else tokens
        trng = np.random.default_rng(46)

        def token():
            h = torch.from_numpy(trng.standard_normal((1, D)).astype(np.float32)).to(device)
            for layer in model.layers:
                layer.mlp(h.to(torch.bfloat16))
                h = h + alpha * torch.from_numpy(
                    trng.standard_normal((1, D)).astype(np.float32)).to(device)

        for _ in range(warm):
            token()
        torch.cuda.synchronize()
        st0 = cache.stats()
        r0 = ring.stats()
        with KernelTimer() as kt:
            c0 = time.perf_counter()
            for _ in range(n_tok):
                token()
            torch.cuda.synchronize()
            wall = time.perf_counter() - c0
        st1 = cache.stats()
        r1 = ring.stats()
        tokens_run = n_tok
        hits = st1["hits"] - st0["hits"]
        misses = st1["misses"] - st0["misses"]
        kern_s = sum(tot for tot, _ in kt.result.values()) / 1e3
        issued = r1["pred_issued"] - r0["pred_issued"]
        used = r1["pred_used"] - r0["pred_used"]
        t = tokens_run
        out[name] = {
            "tokens": t, "tokens_per_s": t / wall, "ms_per_token": wall * 1e3 / t,
            "stall_ms_per_token": max(0.0, wall - kern_s) * 1e3 / t,
            "kernel_ms_per_token": kern_s * 1e3 / t,
            "hit_rate": hits / max(1, hits + misses), "misses_per_token": misses / t,
            "h2d_gb_per_token": (st1["h2d_gb"] - st0["h2d_gb"]) / t,
            "spec_started_per_token": (st1["spec_started"] - st0["spec_started"]) / t,
            "spec_claims_per_token": (st1["spec_claims"] - st0["spec_claims"]) / t,
            "spec_claims_late_per_token": (st1["spec_claims_late"] - st0["spec_claims_late"]) / t,
            "pred_precision": used / issued if issued else None,
        }
        if mode == "auto":
            out[name]["governor"] = ring.governor.describe()
            out[name]["governor_log"] = list(ring.governor.log)
        cache.close()
    store.close()
    out["note"] = ("stall = wall time - sum of kernel times; speculative reads use their own "
                   "copy stream and free slots only; precision = predicted ids routed at the "
                   "target layer / predicted ids")
    return out


def run_qwen3_next(args, device, layers=2):
    """Qwen3-Next-shaped layer (hidden 2048, 512 experts + 1 gated shared
    expert, moe_intermediate 512, top-10 softmax+renorm, 6-bit g64, all
    resident): the 8-token speculative-verify step and a 1024-token prefill,
    each timed as HIP-graph replays over `layers` distinct layers."""
    import torch

    from pagedmoe_amd import kernels as K
    from pagedmoe_amd._lib import KernelTimer, geom
    from pagedmoe_amd.slab import SlabStore

    D, E, I, k = 2048, 512, 512, 10
    g = geom(D, I, 6)
    slots = layers * (E + 1)
    slab = SlabStore(g, slots, device, zero=False)
    gen = torch.Generator(device=device)
    gen.manual_seed(5)
    for slot in range(slots):
        for prefix, rows, cols in (("gate_proj", I, D), ("up_proj", I, D), ("down_proj", D, I)):
            slab.quantize_into(slot, prefix, torch.randn((rows, cols), generator=gen,
                                                         device=device) * 0.02)
    gate = (torch.randn((layers, E, D), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    sgate = (torch.randn((layers, 1, D), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    tables = (torch.arange(layers, device=device, dtype=torch.int32)[:, None] * (E + 1)
              + torch.arange(E, device=device, dtype=torch.int32)[None, :]).contiguous()
    rc = K.route_cfg("softmax", E, k)
    expert_bytes = int(sum(int(g.nbytes[c]) for c in range(9)))
    out = {}
    for name, n in (("verify_8", 8), ("prefill_1024", 1024)):
        x = torch.randn((layers, n, D), generator=gen, device=device).to(torch.bfloat16)
        y = torch.empty((layers, n, D), dtype=torch.bfloat16, device=device)
        inds = torch.empty((layers, n, k), dtype=torch.int32, device=device)
        wts = torch.empty((layers, n, k), dtype=torch.float32, device=device)
        ws = K.moe_workspace(g, n, k, 1, E, device, fresh=True)

        def seq():
            for l in range(layers):
                K.moe_block(g, rc, slab.buf, tables[l], gate[l], x[l], shared_slot=l * (E + 1) + E,
                            shared_gate=sgate[l], out=y[l], inds=inds[l], weights=wts[l], ws=ws)

        seq()
        torch.cuda.synchronize()
        with KernelTimer() as kt:
            seq()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            seq()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            seq()
        graph.replay()
        torch.cuda.synchronize()
        reps = 20 if n <= 8 else 5
        t0 = time.perf_counter()
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / (reps * layers)
        uniq = sum(len(set(inds[l].reshape(-1).tolist())) for l in range(layers)) / layers
        layer_bytes = (uniq + 1) * expert_bytes
        rows = n * (k + 1)
        flops = 2.0 * 3 * D * I * rows
        r = {"tokens": n, "ms_per_step": ms, "tokens_per_s": n / (ms * 1e-3),
             "mean_unique_experts": uniq, "expert_bytes_per_step": layer_bytes,
             "hbm_gbs": layer_bytes / (ms * 1e-3) / 1e9,
             "hbm_frac": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
             "expert_tflops": flops / (ms * 1e-3) / 1e12,
             "mfma_frac": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
             "kernels": {nm: {"avg_us": tot * 1e3 / cnt, "launches": cnt}
                         for nm, (tot, cnt) in kt.result.items()}}
        out[name] = r
    slab.release()
    out["config"] = {"workload": "Qwen3-Next-shaped MoE layer", "hidden": D, "experts": E,
                     "shared_experts": 1, "shared_gate": True, "moe_intermediate": I,
                     "top_k": k, "bits": 6, "group": 64, "layers_cycled": layers}
    return out


def _probe(device):
    import ctypes

    import torch

    from pagedmoe_amd._lib import check, lib

    sink = torch.empty(int(lib().pmoe_probe_sink_bytes()), dtype=torch.uint8, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def read(t, off=0, nbytes=None):
        nbytes = t.numel() - off if nbytes is None else nbytes
        check(lib().pmoe_probe_read(ctypes.c_void_p(t.data_ptr() + off), nbytes,
                                    ctypes.c_void_p(sink.data_ptr()), sink.numel(), stream),
              "pmoe_probe_read")

    def copy(dst, src):
        check(lib().pmoe_probe_copy(ctypes.c_void_p(dst.data_ptr()),
                                    ctypes.c_void_p(src.data_ptr()), src.numel(), stream),
              "pmoe_probe_copy")

    return read, copy


def measured_ceilings(device, layer_bytes):
    """What this box sustains, next to the spec peaks, measured with this
    library's probe kernels (pmoe_probe_read / pmoe_probe_copy, HIP events):
    a 2 GiB streaming read with the expert stream's access pattern; the same
    read over one batch-1 layer's expert volume, cycling 8 disjoint regions
    (more than the 256 MB last-level cache) so no pass finds its bytes in
    cache; a 1 GiB device copy (read + write bytes); and torch.matmul's
    (hipBLASLt) dense bf16 GEMM at the prefill gate/up shape
    (16384 x 4096 x 3072, 412 GFLOP) -- a library figure at one shape, not a
    ceiling for the hand-written kernels."""
    import torch

    read, copy = _probe(device)
    res = {}
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=device)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(2):
        read(buf)
    ev0.record()
    for _ in range(10):
        read(buf)
    ev1.record()
    torch.cuda.synchronize()
    res["hbm_read_gbs"] = buf.numel() * 10 / (ev0.elapsed_time(ev1) * 1e-3) / 1e9
    lb = int(layer_bytes) // 256 * 256
    regions = 8
    for r in range(regions):
        read(buf, r * lb, lb)
    ev0.record()
    for rep in range(40):
        read(buf, (rep % regions) * lb, lb)
    ev1.record()
    torch.cuda.synchronize()
    per = ev0.elapsed_time(ev1) * 1e-3 / 40
    res["layer_volume_read_bytes"] = lb
    res["layer_volume_read_us"] = per * 1e6
    res["layer_volume_read_gbs"] = lb / per / 1e9
    half = buf.numel() // 2
    src, dst = buf[:half], buf[half:]
    copy(dst, src)
    ev0.record()
    for _ in range(10):
        copy(dst, src)
    ev1.record()
    torch.cuda.synchronize()
    res["hbm_copy_gbs"] = 2 * half * 10 / (ev0.elapsed_time(ev1) * 1e-3) / 1e9
    del buf, src, dst
    m, k, n = 16384, 4096, 3072
    a = torch.randn(m, k, device=device, dtype=torch.bfloat16)
    b = torch.randn(n, k, device=device, dtype=torch.bfloat16)
    for _ in range(3):
        c = a @ b.t()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        c = a @ b.t()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / 10
    res["dense_bf16_gemm_tflops"] = 2.0 * m * k * n / dt / 1e12
    res["dense_bf16_gemm_shape"] = [m, k, n]
    res["probe"] = ("pmoe_probe_read: 16-byte non-temporal loads, 1 KB per wave instruction, "
                    "4 loads in flight per lane; pmoe_probe_copy: 16-byte loads and stores")
    del a, b, c
    return res


def pmc_run(args, g, spec, slab, gate, tables, device):
    """Eager layer steps for hardware-counter runs (one dispatch per kernel,
    no graph), followed by a plain copy of known size for calibration."""
    import torch

    from pagedmoe_amd import kernels as K

    E, D, k = spec["experts"], spec["hidden"], spec["top_k"]
    rc = K.route_cfg(spec["scoring"], E, k)
    gen = torch.Generator(device=device)
    gen.manual_seed(2000)
    x = torch.randn((args.steps, args.batch, D), generator=gen, device=device).to(torch.bfloat16)
    ws = K.moe_workspace(g, args.batch, k, 0, E, device, fresh=True)
    inds = torch.empty((args.steps, args.batch, k), dtype=torch.int32, device=device)
    # prefill-sized batches get the skewed router of the prefill workload
    lb = torch.randn((args.layers, E), generator=gen, device=device) if args.batch > 256 else None
    for i in range(args.steps):
        layer = i % args.layers
        K.moe_block(g, rc, slab.buf, tables[layer], gate[layer], x[i], inds=inds[i], ws=ws,
                    logit_bias=None if lb is None else lb[layer])
    torch.cuda.synchronize()
    # calibration in the same process: the probe read of 256 MiB (its
    # FETCH_SIZE against 256 MiB scales that counter) and the probe copy of
    # 256 MiB (its WRITE_SIZE against 256 MiB scales that one)
    read, copy = _probe(device)
    cal = torch.empty(512 << 20, dtype=torch.uint8, device=device)
    read(cal[:256 << 20])
    copy(cal[256 << 20:], cal[:256 << 20])
    torch.cuda.synchronize()
    ids = inds.cpu().numpy().reshape(args.steps, -1)
    uniq = sum(len(set(r.tolist())) for r in ids) / args.steps
    one_launch = ("decode_xcd_kernel" if os.environ.get("PMOE_DECODE_XCD", "1") != "0"
                  else "decode_fused_kernel")
    kernel = "prefill" if args.batch > 256 else (
        one_launch if args.batch == 1 else "gateup_routed_kernel")
    print(json.dumps({"pmc_run": True, "steps": args.steps, "batch": args.batch,
                      "source_hash": source_hash(kernel), "source_kernel": kernel,
                      "mean_unique_experts": uniq, "probe_read_bytes": 256 << 20,
                      "probe_copy_read_bytes": 256 << 20, "probe_copy_write_bytes": 256 << 20,
                      "gateup_bytes_per_step": uniq * 2 * int(g.nbytes[0] + g.nbytes[1] + g.nbytes[2]),
                      "down_bytes_per_step": uniq * int(g.nbytes[6] + g.nbytes[7] + g.nbytes[8])}),
          flush=True)


def cpu_baseline(g, spec, slab, gate, seconds, device):
    """The oracle's C restatement (OpenMP over all host cores) running the
    same decode layer (layer 0's 128 experts, fresh tokens) for ~seconds."""
    import numpy as np
    import torch

    from oracle import c_oracle as C
    from oracle import pmoe_oracle as O

    E = spec["experts"]

    def qt(prefix, slot, cols):
        w = slab.expert(prefix + ".weight", slot).cpu().numpy().view(np.uint32)
        s = slab.expert(prefix + ".scales", slot).cpu().view(torch.int16).numpy().view(np.uint16)
        b = slab.expert(prefix + ".biases", slot).cpu().view(torch.int16).numpy().view(np.uint16)
        return O.QTensor(np.ascontiguousarray(w), np.ascontiguousarray(s),
                         np.ascontiguousarray(b), g.bits, g.group, cols)

    experts = [O.Expert(qt("gate_proj", e, g.hidden), qt("up_proj", e, g.hidden),
                        qt("down_proj", e, g.inter)) for e in range(E)]
    gw = gate[0].cpu().view(torch.int16).numpy().view(np.uint16)
    layer = C.DecodeLayer(gw, experts, g.hidden, g.inter, spec["top_k"], g.bits)
    rng = np.random.default_rng(7)
    layer(O.bf16_round(rng.standard_normal((1, g.hidden), dtype=np.float32)))  # warm
    tokens = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        layer(O.bf16_round(rng.standard_normal((1, g.hidden), dtype=np.float32)))
        tokens += 1
    dt = time.perf_counter() - t0
    return {"value": tokens / dt, "unit": "tokens/s", "cores": C.threads(), "kind": "port",
            "sample": f"{tokens} decode tokens (batch 1) through one Qwen3-235B-shaped MoE layer "
                      f"(128 resident experts, 4-bit g64) in {dt:.1f} s; C restatement of the "
                      f"oracle, OpenMP over {C.threads()} threads; the reference's mlx CPU path "
                      f"is not installable here"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", default="qwen3-235b-decode", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the batch-8 and prefill lines in extra")
    ap.add_argument("--no-paging", action="store_true",
                    help="skip the DeepSeek-shaped paging leg in extra")
    ap.add_argument("--no-predict", action="store_true",
                    help="skip the multi-layer paged decode leg with route prediction")
    ap.add_argument("--no-next", action="store_true",
                    help="skip the Qwen3-Next-shaped (6-bit) leg in extra")
    ap.add_argument("--prefill-reps", type=int, default=5,
                    help="graph replays (of --layers prefill layer steps) timed for the prefill line")
    ap.add_argument("--pmc-run", action="store_true",
                    help="counter-collection run: `--steps` eager layer steps at `--batch`, then "
                         "one 256 MiB device-to-device copy as the counter calibration")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE "
              f"{world}); the expert-parallel split is a design note, not built here.",
              file=sys.stderr, flush=True)
        sys.exit(2)

    import torch

    from pagedmoe_amd._lib import geom

    device = "cuda:0"
    spec = WORKLOADS[args.workload]
    g = geom(spec["hidden"], spec["inter"], spec["bits"])
    log(f"building {args.layers} layers x {spec['experts']} experts "
        f"({args.layers * spec['experts'] * g.expert_bytes / 1e9:.1f} GB)")
    t0 = time.perf_counter()
    slab, gate, tables = build_layers(g, spec, args.layers, device)
    torch.cuda.synchronize()
    log(f"built in {time.perf_counter() - t0:.1f} s")

    if args.pmc_run:
        pmc_run(args, g, spec, slab, gate, tables, device)
        return

    main_res = run_decode(args, g, spec, slab, gate, tables, args.batch, device)
    log(f"batch {args.batch}: {main_res['ms_per_step'] * 1e3:.1f} us/step, "
        f"{main_res['tokens_per_s']:.0f} tok/s, kernels {main_res['kernels']}")
    extra = {}
    if not args.no_extra and args.batch != 8:
        r8 = run_decode(args, g, spec, slab, gate, tables, 8, device)
        log(f"batch 8: {r8['ms_per_step'] * 1e3:.1f} us/step, {r8['tokens_per_s']:.0f} tok/s")
        r8.pop("_gateup_step_bytes", None)
        r8.pop("_layer_bytes", None)
        extra["decode_batch8"] = r8
    if not args.no_extra:
        rp = run_prefill(args, g, spec, slab, gate, tables, device)
        log(f"prefill {rp['tokens']} tokens: {rp['ms_per_step']:.3f} ms/layer, "
            f"{rp['tokens_per_s']:.0f} tok/s, {rp['expert_tflops']:.0f} TFLOP/s "
            f"({100 * rp['mfma_frac_layer']:.1f}% of bf16 MFMA peak), kernels {rp['kernels']}")
        extra["prefill_2048"] = rp
    if not args.no_extra:
        ceil = measured_ceilings(device, main_res["_layer_bytes"])
        log(f"measured ceilings: HBM read {ceil['hbm_read_gbs']:.0f} GB/s (2 GiB), "
            f"{ceil['layer_volume_read_gbs']:.0f} GB/s ({ceil['layer_volume_read_bytes'] / 1e6:.0f}"
            f" MB, {ceil['layer_volume_read_us']:.1f} us), copy {ceil['hbm_copy_gbs']:.0f} GB/s, "
            f"dense bf16 GEMM {ceil['dense_bf16_gemm_tflops']:.0f} TFLOP/s")
        extra["measured_ceilings"] = ceil
        if "prefill_2048" in extra:
            rp = extra["prefill_2048"]
            rp["mfma_frac_of_dense_gemm"] = rp["expert_tflops"] / ceil["dense_bf16_gemm_tflops"]
            for nm in ("prefill_gateup", "prefill_down"):
                kr = rp["kernels"].get(nm)
                if kr and "tflops" in kr:
                    kr["frac_of_dense_gemm"] = kr["tflops"] / ceil["dense_bf16_gemm_tflops"]
    if not args.no_extra and not args.no_next:
        rn = run_qwen3_next(args, device)
        log(f"qwen3-next 6-bit: verify-8 {rn['verify_8']['ms_per_step'] * 1e3:.1f} us/step "
            f"({100 * rn['verify_8']['hbm_frac']:.1f}% HBM), prefill-1024 "
            f"{rn['prefill_1024']['ms_per_step']:.3f} ms/layer "
            f"({100 * rn['prefill_1024']['hbm_frac']:.1f}% HBM, "
            f"{100 * rn['prefill_1024']['mfma_frac']:.1f}% MFMA)")
        extra["qwen3_next_6bit"] = rn
    if not args.no_extra and not args.no_paging:
        rg = run_paging(args, device)
        log(f"deepseek paging: {rg['tokens_per_s']:.0f} tok/s, hit rate {rg['hit_rate']:.3f}, "
            f"stall {rg['stall_ms_per_token']:.3f} ms/token, H2D {rg['h2d_gbs'] or 0:.1f} GB/s")
        extra["deepseek_paging"] = rg
    if not args.no_extra and not args.no_paging and not args.no_predict:
        rp = run_paging_predicted(args, device)
        for nm in ("no_prediction", "prediction", "governor"):
            r = rp[nm]
            log(f"deepseek paged decode, {nm}: {r['ms_per_token']:.2f} ms/token, stall "
                f"{r['stall_ms_per_token']:.2f}, hit rate {r['hit_rate']:.3f}, precision "
                f"{r['pred_precision']} {r.get('governor_log', '')}")
        extra["deepseek_paging_predicted"] = rp

    one_launch = [k for k in ("decode_xcd", "decode_fused") if k in main_res["kernels"]]
    if one_launch:
        kname = one_launch[0] + "_kernel"
        ku = dict(main_res["kernels"][one_launch[0]])
        ku["avg_us"] = ku["graph_avg_us"]  # HIP events over the timed graph replays
        achieved = main_res["fused_gbs"]
        alg = main_res["_layer_bytes"]
        what = (f"{kname} (whole layer in one launch: router, top-k, gate+up+SwiGLU, "
                "down, combine" + (", one pick per XCD)" if kname == "decode_xcd_kernel" else ")"))
    else:
        kname = "gateup_routed_kernel"
        ku = main_res["kernels"]["qgemv_gateup"]
        achieved = main_res["gateup_gbs"]
        alg = main_res["_gateup_step_bytes"]
        what = "gateup_routed_kernel (gate+up+SwiGLU of the routed experts)"
    traffic, traffic_note = load_traffic(f"{args.workload}_b{args.batch}", kname)
    roofline = {"bound": "hbm", "kernel": what,
                "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                "traffic_source": traffic_note,
                "avg_launch_us": ku["avg_us"],
                "algorithmic_bytes_per_launch": alg}
    main_res.pop("_gateup_step_bytes", None)
    main_res.pop("_layer_bytes", None)

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_seconds:.0f} s")
        cpu = cpu_baseline(g, spec, slab, gate, args.cpu_seconds, device)
        log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")

    if "measured_ceilings" in extra:
        mc = extra["measured_ceilings"]
        roofline["frac_of_probe_read_2gib"] = achieved / mc["hbm_read_gbs"]
        roofline["frac_of_probe_read_layer_volume"] = achieved / mc["layer_volume_read_gbs"]
    line = {
        "metric": "MoE-layer tokens/s + % HBM roofline (decode) / % MFMA peak (prefill)",
        "value": main_res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": main_res["steps_timed"],
        "warmup": main_res["untimed_steps"],
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations, 4-bit affine g64 weights, fp32 accumulate",
        "data": "synthetic: N(0,0.02) weights quantized on the GPU, N(0,1) bf16 tokens",
        "config": {"workload": "Qwen3-235B-A22B-shaped MoE layer decode", "hidden": 4096,
                   "experts": 128, "moe_intermediate": 1536, "top_k": 8,
                   "routing": "softmax+renorm", "bits": 4, "group": 64,
                   "batch": args.batch, "layers_cycled": args.layers,
                   "timing": (f"{main_res['graph_replays_timed']} HIP graph replays of "
                              f"{main_res['graph_steps']} layer steps"),
                   "warmup_detail": (f"{args.warmup} eager steps (--warmup), "
                                     f"{main_res['graph_steps']} event-bracketed eager steps, "
                                     f"{main_res['graph_steps']} capture-warm steps, 1 warm "
                                     f"replay of {main_res['graph_steps']}")},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": {"decode": main_res, **extra},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
