#!/usr/bin/env python3
"""Benchmark of the logan-hip decode hot path on one MI355X.

Workload (the metric's "routed-MoE layer at B=1" built
from q4 GEMVs): the Qwen3-Next routed-MoE block at 4-bit g64 — E=512 experts
with gate/up 2048->512 and down 512->2048, top-10 softmax routing with
normalised weights, plus one shared expert of the same shape with its scalar
sigmoid gate — for one token (B=1). A step is one token passing the MoE
blocks of a 48-layer stack whose banks all stay resident in HBM (43.5 GB),
each layer with fresh router logits and activations, so every layer reads
its own 11 experts from HBM and the 256 MB MALL cannot serve repeats. Each
step is one HIP graph of 48 moe_block calls; K graphs are replayed back to
back between two synchronisations.

value = algorithmic bytes per step (48 x 19,477,504 B: packed weights and
bf16 scale/bias of the 11 experts touched, router logits, x, out, shared
gate row) / step time, in GB/s. us_per_token_layer is the same time per
layer. The config-1 q4 GEMV (4096x2048) is timed as a secondary leg over 64
rotated weight copies (302 MB). The CPU baseline is the oracle's
single-threaded restatement of the reference CPU path on a bounded sample
of the same workload.
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

METRIC = "q4 GEMV HBM GB/s (% of 8 TB/s peak); routed-MoE layer us/token at B=1"
PEAK_GBPS = 8000.0

E, TOPK, D, INTER, BITS, GS = 512, 10, 2048, 512, 4, 64


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(O_I_pairs, bits=BITS, gs=GS) -> int:
    return sum(O * I * bits // 8 + 2 * 2 * O * (I // gs) for O, I in O_I_pairs)


PER_EXPERT = expert_bytes([(INTER, D), (INTER, D), (D, INTER)])  # 1,769,472 B
LAYER_BYTES_B1 = (TOPK + 1) * PER_EXPERT + E * 2 + D * 2 + D * 2 + D * 2  # 19,477,504 B
GEMV_O, GEMV_I = 4096, 2048
GEMV_BYTES = GEMV_O * GEMV_I // 2 + 2 * 2 * GEMV_O * (GEMV_I // GS) + GEMV_I * 2 + GEMV_O * 2


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--gemv-launches", type=int, default=2048)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (5 times), to calibrate "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE against known bytes, then exit")
    return ap.parse_args()


def build_layers(torch, device, synth, L):
    layers = []
    for l in range(L):
        s = 1000 * l

        def bank(O, I, n, seed):
            w, sc, bi = synth.torch_affine(O, I, BITS, GS, E=n, seed=seed)
            return device.AffineBank(w, sc, bi, n, O, I, BITS, GS)

        g = torch.Generator(device="cuda")
        g.manual_seed(s + 7)
        se_g = (torch.randn(D, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        layers.append(device.MoeLayer(bank(INTER, D, E, s + 1), bank(INTER, D, E, s + 2),
                                      bank(D, INTER, E, s + 3), TOPK, bank(INTER, D, 1, s + 4),
                                      bank(INTER, D, 1, s + 5), bank(D, INTER, 1, s + 6), se_g))
    return layers


def bench_moe(torch, device, synth, args):
    L = args.layers
    log(f"building {L} resident MoE layers ({L * 0.906:.1f} GB)")
    layers = build_layers(torch, device, synth, L)
    n = args.warmup + args.steps
    g = torch.Generator(device="cuda")
    g.manual_seed(12345)
    xs = torch.randn((n, L, 1, D), device="cuda", generator=g).to(torch.bfloat16)
    logits = torch.randn((n, L, 1, E), device="cuda", generator=g).to(torch.bfloat16)
    out = torch.empty((L, 1, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    # eager pass (checks every layer runs)
    for l in range(L):
        device.moe_block(layers[l], xs[0, l], logits[0, l], out=out[l], workspace=ws)
    torch.cuda.synchronize()
    log("capturing graphs")
    stream = torch.cuda.Stream()
    graphs = []
    for i in range(n):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            for l in range(L):
                device.moe_block(layers[l], xs[i, l], logits[i, l], out=out[l], workspace=ws)
        graphs.append(gr)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            graphs[i].replay()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps x {L} layers")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for i in range(args.warmup, n):
            graphs[i].replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / args.steps
    log(f"moe: {ms_per_step:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f} ms/step)")
    layer_us = ms_per_step * 1e3 / L
    gbps = LAYER_BYTES_B1 * L / (ms_per_step * 1e-3) / 1e9
    del graphs
    cpu_layer = layers[0]
    return dict(ms_per_step=ms_per_step, layer_us=layer_us, gbps=gbps, wall_ms=wall * 1e3 / args.steps,
                layer0=cpu_layer)


def bench_gemv(torch, device, synth, args):
    copies = 64
    mats = []
    for c in range(copies):
        w, sc, bi = synth.torch_affine(GEMV_O, GEMV_I, BITS, GS, seed=50000 + c)
        mats.append(device.AffineMatrix(w, sc, bi, GEMV_O, GEMV_I, BITS, GS))
    x = torch.randn((1, GEMV_I), device="cuda").to(torch.bfloat16)
    y = torch.empty((1, GEMV_O), dtype=torch.bfloat16, device="cuda")
    for m in mats:
        device.affine_gemv(m, x, out=y)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    per_graph = 256
    graphs = []
    for gi in range(max(1, args.gemv_launches // per_graph)):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            for j in range(per_graph):
                device.affine_gemv(mats[(gi * per_graph + j) % copies], x, out=y)
        graphs.append(gr)
    with torch.cuda.stream(stream):
        graphs[0].replay()
    torch.cuda.synchronize()
    launches = len(graphs) * per_graph
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        ev0.record(stream)
        for gr in graphs:
            gr.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / launches
    gbps = GEMV_BYTES / (us * 1e-6) / 1e9
    log(f"gemv q4 4096x2048: {us:.2f} us/launch, {gbps:.0f} GB/s")
    return dict(us_per_launch=us, gbps=gbps, launches=launches)


def measured_traffic():
    """HBM bytes per fused-MoE launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy of known
    size), or None when the summary is absent."""
    f = ROOT / "profiles" / "moe_fused_b1_config3_traffic.json"
    if not f.exists():
        return None
    return json.loads(f.read_text()).get("hbm_bytes_per_launch")


def cpu_baseline(torch, layer, seconds):
    """The oracle (single thread) on tokens of layer 0 until `seconds` pass."""
    import numpy as np

    import oracle

    def host(b):
        return (b.weights.cpu().numpy(), b.scales.cpu().numpy().view(np.uint16),
                b.biases.cpu().numpy().view(np.uint16))

    gate, up, down = host(layer.gate), host(layer.up), host(layer.down)
    shared = tuple(tuple(a[0] for a in host(b)) for b in (layer.shared_gate, layer.shared_up,
                                                          layer.shared_down))
    se_g = layer.shared_gate_vec.float().cpu().numpy()
    rng = np.random.default_rng(0)
    from logan_amd import synth

    n = 0
    t0 = time.perf_counter()
    while True:
        x = synth.bf16_to_f32(synth.make_x(rng, D))
        lg = synth.bf16_to_f32(synth.make_logits(rng, 1, E)[0])
        oracle.moe_token(x, lg, TOPK, D, INTER, BITS, GS, gate, up, down, shared, se_g, nthreads=1)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    us_tok = el / n * 1e6
    return dict(value=LAYER_BYTES_B1 * n / el / 1e9, unit="GB/s", cores=1, kind="port",
                us_per_token_layer=us_tok,
                sample=f"{n} tokens of one config-3 MoE layer (B=1, 4-bit, E=512, top-10 + shared), "
                       f"oracle lo_moe_token, 1 thread, {el:.1f} s")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              f"(the path would shard experts across GPUs; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch

    from logan_amd import backend, device, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    assert backend.hip_init(), "logan-hip failed to initialise"
    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.ones(n // 4, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {args.copy_mib} MiB x 5")
        return
    moe = bench_moe(torch, device, synth, args)
    gemv = None if args.no_gemv else bench_gemv(torch, device, synth, args)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(torch, moe["layer0"], args.cpu_seconds)
        log(f"cpu: {cpu['us_per_token_layer']:.0f} us/token-layer")
    res = {
        "metric": METRIC,
        "value": round(moe["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(moe["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random MLX-affine codes, bf16 |N(0,1)|*0.01 scales, "
                "bias=-8*scale, bf16 N(0,1) activations and router logits)",
        "config": {
            "workload": "config 3: Qwen3-Next routed-MoE layer decode, B=1, 4-bit g64, "
                        "E=512 top-10 + 1 shared expert, D=2048, inter=512; one step = one "
                        f"token through {args.layers} resident layers (fresh routes per layer)",
            "global_batch": 1, "layers_per_step": args.layers, "experts": E, "top_k": TOPK,
            "hidden": D, "inter": INTER, "bits": BITS, "group_size": GS,
            "bytes_per_layer": LAYER_BYTES_B1, "parallelism": "single GPU",
        },
        "us_per_token_layer": round(moe["layer_us"], 3),
        "roofline": {
            "bound": "hbm", "achieved": round(moe["gbps"], 2), "peak": PEAK_GBPS, "unit": "GB/s",
            "frac": round(moe["gbps"] / PEAK_GBPS, 4), "traffic": measured_traffic(),
            "kernel": "moe_fused_b1_kernel: one launch per layer (routing, gate/up + SwiGLU, "
                      "down, rank-ordered combine, shared expert); "
                      f"{LAYER_BYTES_B1} algorithmic B per launch over the event-timed "
                      "average launch interval",
        },
        "cpu_baseline": cpu,
    }
    if gemv:
        res["secondary"] = {"gemv_q4_config1": {
            "shape": "M=1 K=2048 N=4096 4-bit g64", "bytes_per_launch": GEMV_BYTES,
            "us_per_launch": round(gemv["us_per_launch"], 3), "gbps": round(gemv["gbps"], 1),
            "frac_of_peak": round(gemv["gbps"] / PEAK_GBPS, 4), "launches": gemv["launches"],
            "rotation": "64 weight copies (302 MB) > 256 MB MALL"}}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
