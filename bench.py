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

The timed loop replays a HIP graph of `--layers` x 4 consecutive layer steps
(launch overhead excluded, as in the reference's one-graph-per-token decode);
inputs are resident in HBM before timing starts.  A second, eager pass
brackets every kernel with HIP events to give the dominant kernel's average
duration, from which roofline.achieved = algorithmic expert-weight bytes per
launch / that duration.

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


def run_decode(args, g, spec, slab, gate, tables, batch, device):
    import torch

    from pagedmoe_amd import kernels as K
    from pagedmoe_amd._lib import KernelTimer

    E, D, k = spec["experts"], spec["hidden"], spec["top_k"]
    L = args.layers
    seq = L * 4                                   # layer steps per graph
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

    # eager warmup (also validates the call path)
    for _ in range(max(1, args.warmup // seq + 1)):
        run_seq()
    torch.cuda.synchronize()

    # per-kernel durations: eager pass with event brackets
    with KernelTimer() as kt:
        for _ in range(max(1, args.steps // seq)):
            run_seq()
    torch.cuda.synchronize()
    reps_timer = max(1, args.steps // seq)

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
    for _ in range(max(1, args.warmup // seq)):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps // seq)
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    steps_timed = reps * seq
    ms = (t1 - t0) * 1e3 / steps_timed

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
        "tokens_per_s": batch / (ms / 1e3),
        "steps_timed": steps_timed,
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
    kf = res["kernels"].get("decode_fused")
    if kf:
        res["fused_gbs"] = layer_bytes / (kf["avg_us"] * 1e-6) / 1e9
    res["_layer_bytes"] = layer_bytes
    res["layer_expert_gbs"] = res["expert_bytes_per_step"] / (ms * 1e-3) / 1e9
    res["_gateup_step_bytes"] = step_bytes_gu
    del reps_timer
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
    # calibration: one elementwise kernel reading and writing 256 MiB
    src = torch.ones(64 << 20, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    ids = inds.cpu().numpy().reshape(args.steps, -1)
    uniq = sum(len(set(r.tolist())) for r in ids) / args.steps
    print(json.dumps({"pmc_run": True, "steps": args.steps, "batch": args.batch,
                      "mean_unique_experts": uniq, "copy_read_bytes": 256 << 20,
                      "copy_write_bytes": 256 << 20,
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
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--workload", default="qwen3-235b-decode", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the batch-8 and prefill lines in extra")
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

    if "decode_fused" in main_res["kernels"]:
        kname = "decode_fused_kernel"
        ku = main_res["kernels"]["decode_fused"]
        achieved = main_res["fused_gbs"]
        alg = main_res["_layer_bytes"]
        what = ("decode_fused_kernel (whole layer in one launch: router, top-k, gate+up+SwiGLU, "
                "down, combine)")
    else:
        kname = "gateup_routed_kernel"
        ku = main_res["kernels"]["qgemv_gateup"]
        achieved = main_res["gateup_gbs"]
        alg = main_res["_gateup_step_bytes"]
        what = "gateup_routed_kernel (gate+up+SwiGLU of the routed experts)"
    roofline = {"bound": "hbm", "kernel": what,
                "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                "avg_launch_us": ku["avg_us"],
                "algorithmic_bytes_per_launch": alg}
    traffic_file = ROOT / "profiles" / f"traffic_{args.workload}_b{args.batch}.json"
    if traffic_file.exists():
        try:
            tf = json.loads(traffic_file.read_text())
            if tf.get("kernel") == kname:
                roofline["traffic"] = tf.get("bytes_per_launch")
        except (ValueError, OSError):
            pass
    main_res.pop("_gateup_step_bytes", None)
    main_res.pop("_layer_bytes", None)

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_seconds:.0f} s")
        cpu = cpu_baseline(g, spec, slab, gate, args.cpu_seconds, device)
        log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")

    line = {
        "metric": "MoE-layer tokens/s + % HBM roofline (decode) / % MFMA peak (prefill)",
        "value": main_res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": main_res["steps_timed"],
        "warmup": args.warmup,
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
                   "timing": "HIP graph replay of layer steps"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": {"decode": main_res, **extra},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
