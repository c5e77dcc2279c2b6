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

Secondary legs (reported under "secondary", same synthetic scheme, every
one a HIP graph of the product entry points timed with HIP events):
  * config 1: q4 GEMV 4096x2048 over 64 rotated weight copies;
  * config 2: dense 8-bit g64 decode layer (QKV 4096->6144, O 4096->4096,
    gate/up 4096->14336 with its SwiGLU, down 14336->4096) at M = 1, 4, 8 over 4
    rotated layers (927 MB); and the whole Llama decode layer (norms, RoPE,
    attention over 256 cached tokens, residuals) at M = 1 for affine-8 and
    bf16 weights;
  * MXFP4 (fmt 7): the config-1-shaped GEMV and a 16-matrix batch;
  * config 3 at B = 16 (and 32) over the 48 resident layers, distinct
    experts U counted from the routes;
  * config 4: 5-bit and 6-bit layers with Zipf(1.1) router logits at B = 1
    and B = 32 over 16 resident layers per width;
  * config 5: the 48-layer Qwen3-Next-80B-A3B stack (12 full-attention
    layers with q/k/v/o projections, 36 linear-attention layers with
    qkvz/ba/out projections, every layer with its MoE block), decode B = 1
    and B = 32, and a prefill chunk of M = 512 (projections on the MFMA
    product, MoE block in chunks of 64 tokens). The attention / recurrence
    math between the projections is outside the path: its inputs are
    synthetic activations of the right shape;
  * loader: one config-3 layer's switch_mlp banks (906 MB) from a
    safetensors file into HBM, whole banks and one expert at a time;
  * expert cache: the same banks served by the route-driven expert cache
    (route on device, route to the host, fetch, block on cached experts)
    cold (every rank streamed) and warm (every rank retained).
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
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--legs",
                    default="gemv,dense8,llama,moe3,stack5,moe4,dropin,router,mxfp4,loader,cache",
                    help="secondary legs to run (comma list of gemv, dense8, llama, moe3, stack5, "
                         "moe4, dropin, router, mxfp4, loader, cache; 'none' for none)")
    ap.add_argument("--no-gemv", action="store_true", help="skip the config-1 GEMV leg")
    ap.add_argument("--no-secondary", action="store_true", help="same as --legs none")
    ap.add_argument("--reps", type=int, default=5, help="graph replays per secondary measurement")
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


def bench_moe(torch, device, synth, args, layers):
    L = args.layers
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
    return dict(ms_per_step=ms_per_step, layer_us=layer_us, gbps=gbps, wall_ms=wall * 1e3 / args.steps)


def graph_us(torch, step, reps):
    """Capture step() (launches on the current stream) once into a HIP graph,
    replay it once untimed, then `reps` times between two HIP events on the
    capture stream; microseconds per replay."""
    step()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        step()
    with torch.cuda.stream(stream):
        gr.replay()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(reps):
            gr.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    del gr
    return ev0.elapsed_time(ev1) * 1e3 / reps


def distinct_experts(logits_bf16_bits, k):
    """Distinct experts over a batch's top-k routes (softmax is monotone, so
    the top-k of the logits with lower-index ties; stable sort)."""
    import numpy as np

    lg = (logits_bf16_bits.astype(np.uint32) << 16).view(np.float32)
    top = np.argsort(-lg, axis=-1, kind="stable")[..., :k]
    return len(np.unique(top))


def dev_bf16(torch, bits):
    import numpy as np

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def moe_batch_leg(torch, device, synth, layers, B, bits, per_expert, zipf, reps, seed):
    """One graph step = B tokens through every layer of `layers` (fresh x and
    logits per layer); algorithmic bytes per layer = (U + 1) experts (U
    distinct routed, plus the shared one) + logits + x + out + gate row."""
    import numpy as np

    rng = np.random.default_rng(seed)
    n = len(layers)
    lgb = [synth.make_logits(rng, B, E, zipf) for _ in range(n)]
    xs = [dev_bf16(torch, synth.make_x(rng, B, D)) for _ in range(n)]
    lg = [dev_bf16(torch, a) for a in lgb]
    out = torch.empty((B, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(layers[0].workspace_bytes(B), dtype=torch.uint8, device="cuda")

    def step():
        for l in range(n):
            device.moe_block(layers[l], xs[l], lg[l], out=out, workspace=ws)

    us = graph_us(torch, step, reps) / n
    U = float(np.mean([distinct_experts(a, TOPK) for a in lgb]))
    nbytes = (U + 1) * per_expert + B * (E * 2 + 3 * D * 2)
    return dict(B=B, bits=bits, us_per_layer=round(us, 2), us_per_token_layer=round(us / B, 3),
                distinct_experts=round(U, 1), bytes_per_layer=int(nbytes),
                gbps=round(nbytes / (us * 1e-6) / 1e9, 1),
                frac_of_peak=round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBPS, 4), layers=n,
                router="Zipf(%.1f)" % zipf if zipf else "N(0,1)")


def build_moe_layers(torch, device, synth, n, bits, seed0):
    per = []
    for l in range(n):
        s = seed0 + 1000 * l

        def bank(O, I, ne, seed):
            w, sc, bi = synth.torch_affine(O, I, bits, GS, E=ne, seed=seed)
            return device.AffineBank(w, sc, bi, ne, O, I, bits, GS)

        g = torch.Generator(device="cuda")
        g.manual_seed(s + 7)
        se_g = (torch.randn(D, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        per.append(device.MoeLayer(bank(INTER, D, E, s + 1), bank(INTER, D, E, s + 2),
                                   bank(D, INTER, E, s + 3), TOPK, bank(INTER, D, 1, s + 4),
                                   bank(INTER, D, 1, s + 5), bank(D, INTER, 1, s + 6), se_g))
    return per


def bench_config4(torch, device, synth, args):
    res = {}
    for bits in (5, 6):
        per_expert = expert_bytes([(INTER, D), (INTER, D), (D, INTER)], bits)
        n = 16
        log(f"config 4: building {n} {bits}-bit layers")
        layers = build_moe_layers(torch, device, synth, n, bits, 7_000_000 * bits)
        for B in (1, 32):
            r = moe_batch_leg(torch, device, synth, layers, B, bits, per_expert, 1.1, args.reps,
                              seed=bits * 100 + B)
            log(f"config 4 {bits}-bit B={B}: {r['us_per_layer']} us/layer, {r['gbps']} GB/s, "
                f"U={r['distinct_experts']}")
            res[f"b{bits}_B{B}"] = r
        del layers
        torch.cuda.empty_cache()
    return res


DENSE_H, DENSE_Q, DENSE_F = 4096, 6144, 14336
DENSE8_LAYER_BYTES = expert_bytes([(DENSE_Q, DENSE_H), (DENSE_H, DENSE_H), (DENSE_F, DENSE_H),
                                   (DENSE_F, DENSE_H), (DENSE_H, DENSE_F)], 8)  # 231,735,296 B


def bench_config2(torch, device, synth, args):
    """Dense 8-bit decode layer: QKV, O, gate, up, SwiGLU, down. The O input
    stands in for the attention output (outside the path)."""
    nl = 4
    log(f"config 2: building {nl} dense 8-bit layers ({nl * DENSE8_LAYER_BYTES / 1e9:.2f} GB)")
    shapes = (("qkv", DENSE_Q, DENSE_H), ("o", DENSE_H, DENSE_H), ("gate", DENSE_F, DENSE_H),
              ("up", DENSE_F, DENSE_H), ("down", DENSE_H, DENSE_F))
    layers = []
    for l in range(nl):
        m = {}
        for j, (name, O, I) in enumerate(shapes):
            w, sc, bi = synth.torch_affine(O, I, 8, GS, seed=900_000 + 10 * l + j)
            m[name] = device.AffineMatrix(w, sc, bi, O, I, 8, GS)
        layers.append(m)
    res = {}
    for M in getattr(args, "dense_m", (1, 4, 8)):
        g = torch.Generator(device="cuda")
        g.manual_seed(M)
        x = torch.randn((M, DENSE_H), device="cuda", generator=g).to(torch.bfloat16)
        att = torch.randn((M, DENSE_H), device="cuda", generator=g).to(torch.bfloat16)
        qkv = torch.empty((M, DENSE_Q), dtype=torch.bfloat16, device="cuda")
        o = torch.empty((M, DENSE_H), dtype=torch.bfloat16, device="cuda")
        gt = torch.empty((M, DENSE_F), dtype=torch.bfloat16, device="cuda")
        up = torch.empty((M, DENSE_F), dtype=torch.bfloat16, device="cuda")
        y = torch.empty((M, DENSE_H), dtype=torch.bfloat16, device="cuda")

        def step():
            for L in layers:
                device.affine_gemv(L["qkv"], x, out=qkv)
                device.affine_gemv(L["o"], att, out=o)
                # gate+up: the config's 4096 -> 2 x 14336 projection and its
                # SwiGLU as one product of the two matrices that share x
                device.affine_gemv_swiglu(L["gate"], L["up"], o, out=gt)
                device.affine_gemv(L["down"], gt, out=y)

        us = graph_us(torch, step, args.reps) / nl
        nbytes = DENSE8_LAYER_BYTES + 139_264 * M
        gbps = nbytes / (us * 1e-6) / 1e9
        log(f"config 2 M={M}: {us:.2f} us/layer, {gbps:.0f} GB/s")
        res[f"M{M}"] = dict(us_per_layer=round(us, 2), bytes_per_layer=nbytes, gbps=round(gbps, 1),
                            frac_of_peak=round(gbps / PEAK_GBPS, 4))
    res["layers_rotated"] = nl
    del layers
    torch.cuda.empty_cache()
    return res


DENSE_HEADS, DENSE_KV_HEADS, DENSE_HD, DENSE_CTX = 32, 8, 128, 256


def bench_llama(torch, device, synth, args):
    """Config 2 as the reference runs it at decode: the whole dense Llama layer
    (coli_metal_llama_layer's device form, logan_hip_llama_layer) with
    RMSNorms, RoPE, attention over a 256-token f32 K/V cache, residuals and
    SwiGLU, for affine-8 g64 weights (fmt 15) and for the loader's bf16
    weights (fmt 5), over 4 rotated layers each."""
    nl, pos = 4, DENSE_CTX - 1
    qd, kvd = DENSE_HEADS * DENSE_HD, DENSE_KV_HEADS * DENSE_HD
    shapes = ((qd, DENSE_H), (kvd, DENSE_H), (kvd, DENSE_H), (DENSE_H, qd), (DENSE_F, DENSE_H),
              (DENSE_F, DENSE_H), (DENSE_H, DENSE_F))
    res = {"context_tokens": DENSE_CTX, "layers_rotated": nl}
    for fmt in (15, 5):
        layers = []
        wbytes = 0
        for l in range(nl):
            mats = []
            for j, (O, I) in enumerate(shapes):
                if fmt == 15:
                    w, sc, bi = synth.torch_affine(O, I, 8, GS, seed=700_000 + 10 * l + j)
                    mats.append(device.DenseMatrix(w, O, I, 15, sc, bi))
                    wbytes += O * I + 4 * O * (I // GS)
                else:
                    g = torch.Generator(device="cuda")
                    g.manual_seed(710_000 + 10 * l + j)
                    w = (torch.randn((O, I), device="cuda", generator=g) / (I ** 0.5)).to(torch.bfloat16)
                    mats.append(device.DenseMatrix(w.view(torch.int16), O, I, 5))
                    wbytes += O * I * 2
            g = torch.Generator(device="cuda")
            g.manual_seed(720_000 + l)
            kc = torch.randn((DENSE_CTX, kvd), device="cuda", generator=g)
            vc = torch.randn((DENSE_CTX, kvd), device="cuda", generator=g)
            ones = torch.ones(DENSE_H, device="cuda")
            layers.append(device.LlamaLayer(mats, ones, ones, kc, vc, DENSE_H, DENSE_F, DENSE_HEADS,
                                            DENSE_KV_HEADS, DENSE_HD, 500000.0, 1e-5))
        x = torch.randn(DENSE_H, device="cuda")
        ws = torch.empty(device.llama_workspace_bytes(layers[0], pos), dtype=torch.uint8,
                         device="cuda")

        def step():
            for L in layers:
                device.llama_layer(L, x, pos, workspace=ws)

        us = graph_us(torch, step, args.reps) / nl
        nbytes = wbytes // nl + 2 * DENSE_CTX * kvd * 4 + 2 * DENSE_H * 4
        gbps = nbytes / (us * 1e-6) / 1e9
        name = "affine8_fmt15" if fmt == 15 else "bf16_fmt5"
        log(f"llama layer {name}: {us:.2f} us/layer, {gbps:.0f} GB/s")
        res[name] = dict(us_per_layer=round(us, 2), bytes_per_layer=nbytes, gbps=round(gbps, 1),
                         frac_of_peak=round(gbps / PEAK_GBPS, 4))
        del layers
        torch.cuda.empty_cache()
    return res


def bench_mxfp4(torch, device, args):
    """MXFP4 (fmt 7) GEMV at the config-1 shape (4096 x 2048) over 64 rotated
    copies, and 16 expert-shaped matrices (512 x 2048) with their own x in
    one launch over 16 rotated sets."""
    O, I, copies = GEMV_O, GEMV_I, 64
    mats = []
    for c in range(copies):
        g = torch.Generator(device="cuda")
        g.manual_seed(800_000 + c)
        codes = torch.randint(0, 256, (O, I // 2), dtype=torch.uint8, device="cuda", generator=g)
        sc = torch.randint(118, 136, (O, I // 32), dtype=torch.uint8, device="cuda", generator=g)
        mats.append(device.Mxfp4Matrix(codes, sc, O, I))
    x = torch.randn(I, device="cuda").to(torch.bfloat16)
    y = torch.empty(O, dtype=torch.bfloat16, device="cuda")

    def step():
        for m in mats:
            device.mxfp4_gemv([m], [x], outs=[y])

    us = graph_us(torch, step, args.reps) / copies
    nbytes = O * I // 2 + O * I // 32 + I * 2 + O * 2
    gbps = nbytes / (us * 1e-6) / 1e9
    log(f"mxfp4 gemv 4096x2048: {us:.2f} us/launch, {gbps:.0f} GB/s")
    res = {"gemv_4096x2048": dict(us_per_launch=round(us, 3), bytes_per_launch=nbytes,
                                  gbps=round(gbps, 1), frac_of_peak=round(gbps / PEAK_GBPS, 4),
                                  rotation="64 copies (285 MB)")}
    sets = []
    for s_ in range(16):
        ms = []
        for e in range(16):
            g = torch.Generator(device="cuda")
            g.manual_seed(810_000 + 16 * s_ + e)
            codes = torch.randint(0, 256, (INTER, D // 2), dtype=torch.uint8, device="cuda", generator=g)
            sc = torch.randint(118, 136, (INTER, D // 32), dtype=torch.uint8, device="cuda", generator=g)
            ms.append(device.Mxfp4Matrix(codes, sc, INTER, D))
        sets.append(ms)
    xs = [torch.randn(D, device="cuda") for _ in range(16)]
    ys = [torch.empty(INTER, device="cuda") for _ in range(16)]

    def step16():
        for ms in sets:
            device.mxfp4_gemv(ms, xs, outs=ys)

    us16 = graph_us(torch, step16, args.reps) / len(sets)
    nb16 = 16 * (INTER * D // 2 + INTER * D // 32 + D * 4 + INTER * 4)
    g16 = nb16 / (us16 * 1e-6) / 1e9
    log(f"mxfp4 16 x 512x2048 (f32 x): {us16:.2f} us/launch, {g16:.0f} GB/s")
    res["batch16_512x2048_f32x"] = dict(us_per_launch=round(us16, 3), bytes_per_launch=nb16,
                                        gbps=round(g16, 1), frac_of_peak=round(g16 / PEAK_GBPS, 4))
    del mats, sets
    torch.cuda.empty_cache()
    return res


def bench_loader(torch, args):
    """Checkpoint -> HBM: one config-3 layer's stacked switch_mlp banks
    (gate/up/down, 512 experts, 4-bit g64, 906 MB) written as a safetensors
    file, then made resident by logan_hip_load_mlx_quantized_experts (three
    whole-bank transfers), and the reference's per-expert form (one call per
    (expert, role), 10 experts of a route). The file was just written, so the
    page cache holds it: this is the host-memory -> HBM rate, set beside a
    plain pinned host -> device copy of the same size."""
    import tempfile

    import numpy as np

    from safetensors.numpy import save_file

    from logan_amd import checkpoint

    rng = np.random.default_rng(77)
    tensors = {}
    for role, O, I in (("gate_proj", INTER, D), ("up_proj", INTER, D), ("down_proj", D, INTER)):
        words = I * BITS // 32
        tensors[f"model.layers.0.mlp.switch_mlp.{role}.weight"] = rng.integers(
            0, 2**32, (E, O, words), dtype=np.uint32)
        for part in ("scales", "biases"):
            # fp16 sidecars (the F16 form load_mlx_quantized_* accepts)
            tensors[f"model.layers.0.mlp.switch_mlp.{role}.{part}"] = rng.integers(
                0, 2**16, (E, O, I // GS), dtype=np.uint16).view(np.float16)
    total = sum(a.nbytes for a in tensors.values())
    tmpdir = os.environ.get("TMPDIR", "/tmp")
    fd, path = tempfile.mkstemp(suffix=".safetensors", dir=tmpdir)
    os.close(fd)
    try:
        save_file(tensors, path)
        del tensors
        roles = (("gate_proj", INTER, D), ("up_proj", INTER, D), ("down_proj", D, INTER))
        with checkpoint.StFile.open(path) as st:
            times = []
            for rep in range(4):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                banks = [checkpoint.load_mlx_quantized_bank(st, f"model.layers.0.mlp.switch_mlp."
                                                            f"{r}.weight", E, O, I)
                         for r, O, I in roles]
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                del banks
            bank_s = sorted(times[1:])[1]  # median of the 3 after the first
            ex = rng.choice(E, TOPK, replace=False)
            ts = []
            for rep in range(4):
                t0 = time.perf_counter()
                held = [checkpoint.load_mlx_quantized_expert_wt(
                    st, f"model.layers.0.mlp.switch_mlp.{r}.weight", int(e), E, O, I)
                    for e in ex for r, O, I in roles]
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t0)
                del held
            ex_s = sorted(ts[1:])[1]
    finally:
        os.unlink(path)
    n = 256 << 20
    h = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    dbuf = torch.empty(n, dtype=torch.uint8, device="cuda")
    cts = []
    for _ in range(4):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dbuf.copy_(h, non_blocking=True)
        torch.cuda.synchronize()
        cts.append(time.perf_counter() - t0)
    copy_gbps = n / sorted(cts[1:])[1] / 1e9
    gbps = total / bank_s / 1e9
    log(f"loader: 3 banks {total / 1e6:.0f} MB in {bank_s * 1e3:.1f} ms = {gbps:.1f} GB/s "
        f"(pinned copy {copy_gbps:.1f} GB/s); 30 one-expert loads {ex_s * 1e3:.2f} ms")
    del h, dbuf
    torch.cuda.empty_cache()
    return dict(bytes=total, banks_ms=round(bank_s * 1e3, 2), gbps=round(gbps, 2),
                pinned_h2d_copy_gbps=round(copy_gbps, 2),
                frac_of_pinned_copy=round(gbps / copy_gbps, 3),
                one_expert_loads=dict(calls=3 * TOPK, ms=round(ex_s * 1e3, 3),
                                      bytes=TOPK * PER_EXPERT,
                                      gbps=round(TOPK * PER_EXPERT / ex_s / 1e9, 2)),
                source="page cache (file just written); median of 3 after one warm-up")


def bench_cache(torch, device, synth, args, layers):
    """Route-driven expert cache (logan_hip_expert_cache_*, the reference's
    RouteCache / RouteArena) at config 3: one layer's switch_mlp banks
    (512 experts, 4-bit g64, fp16 sidecars) in a safetensors file, the
    shared expert resident. Per token-layer, wall time of what an engine
    does on this path: route on device (logan_hip_route_topk), the route to
    the host (one synchronisation), fetch (cache bookkeeping plus the loads
    of missed and arena ranks from the file through the pinned staging ring
    into HBM, ordered before the block), the block on the cached experts,
    then a synchronisation. cold: no retained blocks, every rank streams
    through the route arena (10 experts, 17.7 MB per token-layer, from the
    page cache); warm: 10 retained blocks and one route repeated, every
    rank hits; resident: the same route / sync / block sequence on resident
    banks (no fetch), the floor of the host round trip."""
    import tempfile

    import numpy as np

    from safetensors.numpy import save_file

    from logan_amd import checkpoint

    rng = np.random.default_rng(88)
    tensors = {}
    for role, O, I in (("gate_proj", INTER, D), ("up_proj", INTER, D), ("down_proj", D, INTER)):
        w, sc, bi = synth.make_affine(rng, O, I, BITS, GS, fp16=True, E=E)
        tensors[f"model.layers.0.mlp.switch_mlp.{role}.weight"] = w.view(np.uint32)
        tensors[f"model.layers.0.mlp.switch_mlp.{role}.scales"] = sc.view(np.float16)
        tensors[f"model.layers.0.mlp.switch_mlp.{role}.biases"] = bi.view(np.float16)
    tmpdir = os.environ.get("TMPDIR", "/tmp")
    fd, path = tempfile.mkstemp(suffix=".safetensors", dir=tmpdir)
    os.close(fd)
    res = {}
    try:
        save_file(tensors, path)
        del tensors
        n = 40
        g = torch.Generator(device="cuda")
        g.manual_seed(4242)
        xs = torch.randn((n, 1, D), device="cuda", generator=g).to(torch.bfloat16)
        lgs = torch.randn((n, 1, E), device="cuda", generator=g).to(torch.bfloat16)
        out = torch.empty((1, D), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
        base = layers[0]
        with checkpoint.StFile.open(path) as st:
            for mode, blocks, same in (("cold", 0, False), ("warm", TOPK, True)):
                cache = checkpoint.ExpertCache(st, E, D, INTER, blocks_per_layer=blocks, topk=TOPK,
                                               layers=1)
                lay = device.MoeLayer(*cache.geometry(BITS, GS, aux_fp16=True), TOPK,
                                      base.shared_gate, base.shared_up, base.shared_down,
                                      base.shared_gate_vec)

                def token(i):
                    j = 0 if same else i
                    idx, _ = device.route_topk(lgs[j], TOPK)
                    ex = idx.cpu().numpy()[0]
                    bl = cache.fetch(0, ex)
                    device.moe_block_cached(lay, cache, ex, bl, xs[i], lgs[j], out=out, workspace=ws)

                for i in range(3):
                    token(i)
                torch.cuda.synchronize()
                s0 = cache.stats()
                t0 = time.perf_counter()
                for i in range(3, n):
                    token(i)
                torch.cuda.synchronize()
                us = (time.perf_counter() - t0) / (n - 3) * 1e6
                s1 = cache.stats()
                loaded = s1["bytes_loaded"] - s0["bytes_loaded"]
                res[mode] = dict(us_per_token_layer=round(us, 1),
                                 hits=s1["hits"] - s0["hits"], misses=s1["misses"] - s0["misses"],
                                 streamed=s1["streamed"] - s0["streamed"],
                                 bytes_loaded_per_token=loaded // (n - 3),
                                 load_gbps=round(loaded / (us * 1e-6 * (n - 3)) / 1e9, 2))
                log(f"expert cache {mode}: {us:.1f} us/token-layer, {res[mode]}")
                cache.close()
        # the same host round trip on resident banks
        for i in range(3):
            idx, _ = device.route_topk(lgs[i], TOPK)
            idx.cpu()
            device.moe_block(base, xs[i], lgs[i], out=out, workspace=ws)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(3, n):
            idx, _ = device.route_topk(lgs[i], TOPK)
            idx.cpu()
            device.moe_block(base, xs[i], lgs[i], out=out, workspace=ws)
        torch.cuda.synchronize()
        res["resident"] = dict(us_per_token_layer=round((time.perf_counter() - t0) / (n - 3) * 1e6, 1))
        log(f"expert cache resident floor: {res['resident']}")
    finally:
        os.unlink(path)
    res["block_bytes"] = PER_EXPERT
    res["source"] = "page cache (file just written); wall time per token-layer, 37 tokens"
    return res


# Qwen3-Next-80B-A3B projections per layer (hidden 2048; 16 q heads x 256 with
# the output gate, 2 kv heads x 256; linear attention 16 k heads x 128,
# 32 v heads x 128): (name, O, I)
FULL_ATTN = (("q", 8192, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 4096))
LIN_ATTN = (("qkvz", 12288, 2048), ("ba", 64, 2048), ("out", 2048, 4096))
FULL_EVERY = 4


def bench_config5(torch, device, synth, args, moe_layers):
    """48-layer stack: per layer its attention projections (4-bit g64) plus
    its MoE block. Layers l % 4 == 3 are full attention."""
    import numpy as np

    nl = len(moe_layers)
    log(f"config 5: building {nl} layers of attention projections")
    proj = []
    pbytes = 0
    pflop_per_tok = 0
    for l in range(nl):
        shapes = FULL_ATTN if l % FULL_EVERY == FULL_EVERY - 1 else LIN_ATTN
        m = []
        for j, (name, O, I) in enumerate(shapes):
            w, sc, bi = synth.torch_affine(O, I, BITS, GS, seed=5_000_000 + 10 * l + j)
            m.append(device.AffineMatrix(w, sc, bi, O, I, BITS, GS))
            pbytes += expert_bytes([(O, I)])
            pflop_per_tok += 2 * O * I
        proj.append(m)
    moe_bytes_b1 = nl * (TOPK + 1) * PER_EXPERT
    res = {"layers": nl, "projection_bytes": pbytes}
    rng = np.random.default_rng(55)
    for B in (1, 32):
        x = dev_bf16(torch, synth.make_x(rng, B, D))
        att = dev_bf16(torch, synth.make_x(rng, B, 4096))
        lgb = [synth.make_logits(rng, B, E) for _ in range(nl)]
        lg = [dev_bf16(torch, a) for a in lgb]
        outs = {}
        for shapes in (FULL_ATTN, LIN_ATTN):
            for name, O, I in shapes:
                outs[name] = torch.empty((B, O), dtype=torch.bfloat16, device="cuda")
        mo = torch.empty((B, D), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(moe_layers[0].workspace_bytes(B), dtype=torch.uint8, device="cuda")
        def step():
            for l in range(nl):
                shapes = FULL_ATTN if l % FULL_EVERY == FULL_EVERY - 1 else LIN_ATTN
                # the projections that read the hidden state share one launch
                # (q/k/v, qkvz/ba); the output projection reads the attention
                # output
                grp = [(m, outs[name]) for (name, O, I), m in zip(shapes, proj[l]) if I == D]
                device.affine_gemv_multi([m for m, _ in grp], x, outs=[o for _, o in grp])
                for (name, O, I), m in zip(shapes, proj[l]):
                    if I != D:
                        device.affine_gemv(m, att, out=outs[name])
                device.moe_block(moe_layers[l], x, lg[l], out=mo, workspace=ws)

        us = graph_us(torch, step, args.reps)
        U = [distinct_experts(a, TOPK) for a in lgb]
        nbytes = pbytes + sum((u + 1) * PER_EXPERT for u in U)
        gbps = nbytes / (us * 1e-6) / 1e9
        log(f"config 5 decode B={B}: {us:.1f} us/step, {us / B:.2f} us/token, {gbps:.0f} GB/s")
        res[f"decode_B{B}"] = dict(us_per_step=round(us, 1), us_per_token=round(us / B, 2),
                                   bytes_per_step=int(nbytes), gbps=round(gbps, 1),
                                   frac_of_peak=round(gbps / PEAK_GBPS, 4),
                                   projections="affine_gemv_multi (q/k/v, qkvz/ba) + affine_gemv")
    # prefill chunk: M = 512 tokens
    M = 512
    x = dev_bf16(torch, synth.make_x(rng, M, D))
    att = dev_bf16(torch, synth.make_x(rng, M, 4096))
    outs = {}
    for shapes in (FULL_ATTN, LIN_ATTN):
        for name, O, I in shapes:
            outs[name] = torch.empty((M, O), dtype=torch.bfloat16, device="cuda")

    def proj_step():
        for l in range(nl):
            shapes = FULL_ATTN if l % FULL_EVERY == FULL_EVERY - 1 else LIN_ATTN
            # the projections of the hidden state share one product launch
            # (q/k/v, qkvz/ba), the output projection reads the attention output
            grp = [(m, outs[name]) for (name, O, I), m in zip(shapes, proj[l]) if I == D]
            device.affine_qmm_multi([m for m, _ in grp], x, outs=[o for _, o in grp])
            for (name, O, I), m in zip(shapes, proj[l]):
                if I != D:
                    device.affine_qmm(m, att, out=outs[name])

    us_p = graph_us(torch, proj_step, args.reps)
    tflops = pflop_per_tok * M / (us_p * 1e-6) / 1e12
    lgb = [synth.make_logits(rng, M, E) for _ in range(nl)]
    lg = [dev_bf16(torch, a) for a in lgb]
    mo = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(moe_layers[0].workspace_bytes(M), dtype=torch.uint8, device="cuda")

    def moe_step():
        for l in range(nl):
            device.moe_block(moe_layers[l], x, lg[l], out=mo, workspace=ws)

    us_m = graph_us(torch, moe_step, max(1, args.reps // 2))
    log(f"config 5 prefill M={M}: projections {us_p:.0f} us ({tflops:.1f} TFLOP/s), "
        f"MoE {us_m:.0f} us")
    res["prefill_M512"] = dict(
        projections_us=round(us_p, 1), projections_tflops=round(tflops, 2),
        projections_frac_of_bf16_mfma_peak=round(tflops / 2500.0, 4),
        projection_flop=pflop_per_tok * M, moe_us=round(us_m, 1),
        moe_bytes=int(sum((distinct_experts(a, TOPK) + 1) * PER_EXPERT for a in lgb)),
        us_per_chunk=round(us_p + us_m, 1), tokens_per_s=round(M / ((us_p + us_m) * 1e-6), 1))
    res["moe_bytes_b1_ideal"] = moe_bytes_b1
    del proj
    torch.cuda.empty_cache()
    return res


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


def bench_router(torch, device, synth, args, layers):
    """Config 3, B = 1, with the router on device (logan_hip_moe_block_routed):
    per layer the 512 x 2048 router GEMV (8-bit g64, as MLX checkpoints keep
    routers) writes f32 logits and the single-launch block routes on them
    (logan-qwen4/src/lib.rs:7990-7991). Same graph-replay timing as the
    headline; bytes add the router matrix and the f32 logits written and
    read, and drop the bf16 logits the headline reads."""
    L = args.layers
    n = args.warmup + args.steps
    routers = []
    for l in range(L):
        w, sc, bi = synth.torch_affine(E, D, 8, GS, seed=7_000_000 + l)
        # scales |N(0,1)| * 4e-4: logits of x ~ N(0,1) come out near N(0,1),
        # the scale of real router logits
        sc = (sc.view(torch.bfloat16).float() * 0.04).to(torch.bfloat16).view(torch.int16)
        bi = (sc.view(torch.bfloat16).float() * -128).to(torch.bfloat16).view(torch.int16)
        routers.append(device.AffineMatrix(w, sc, bi, E, D, 8, GS))
    g = torch.Generator(device="cuda")
    g.manual_seed(54321)
    xs = torch.randn((n, L, 1, D), device="cuda", generator=g).to(torch.bfloat16)
    out = torch.empty((L, 1, D), dtype=torch.bfloat16, device="cuda")
    lg = torch.empty((L, 1, E), dtype=torch.float32, device="cuda")
    ws = torch.empty(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")

    def step(i):
        for l in range(L):
            device.moe_block_routed(layers[l], routers[l], xs[i, l], out=out[l], logits=lg[l],
                                    workspace=ws)

    step(0)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graphs = []
    for i in range(n):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            step(i)
        graphs.append(gr)
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            graphs[i].replay()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for i in range(args.warmup, n):
            graphs[i].replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / args.steps / L
    router_bytes = E * D + 2 * 2 * E * (D // GS)
    nbytes = LAYER_BYTES_B1 - E * 2 + router_bytes + 2 * E * 4
    log(f"config 3 B=1 with the router on device: {us:.2f} us/layer")
    del graphs
    return dict(us_per_layer=round(us, 2), bytes_per_layer=nbytes,
                gbps=round(nbytes / (us * 1e-6) / 1e9, 1),
                frac_of_peak=round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBPS, 4), layers=L,
                launches_per_layer=2, router="512 x 2048, 8-bit g64, f32 logits")


def bench_dropin(torch, synth, args):
    """The host-pointer drop-in layer, called the way logan-metal's engines
    call it (host f32 activations and outputs, weights cached behind tensor
    handles after the first call): config 1 through coli_metal_matmul, and a
    config-3 B=1 layer through coli_metal_moe_route_begin -> the shared
    expert (between begin and finish, as the reference's caller does) ->
    finish, with the caller's own softmax top-10 and rank-ordered combine on
    the host (logan-qwen4/src/lib.rs:7993-8043, :8692-8711). Each figure is
    wall-clock per call (PCIe copies and synchronisation included) and device
    time only (the library's profile counters: events around the kernels)."""
    import ctypes as C

    import numpy as np
    from logan_amd import _lib as L
    from logan_amd import backend

    lib = L.lib()
    lib.coli_metal_matmul.restype = C.c_int32
    lib.coli_metal_matmul.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                      C.c_int32]
    rng = np.random.default_rng(77)
    res = {}
    # ---- config 1
    w, sc, bi = synth.make_affine(rng, GEMV_O, GEMV_I, BITS, GS)
    aux = synth.aux_bytes(sc, bi)
    x = synth.bf16_to_f32(synth.make_x(rng, GEMV_I))
    y = np.zeros(GEMV_O, np.float32)
    t = C.c_void_p()
    assert lib.coli_metal_matmul(C.byref(t), y.ctypes.data, x.ctypes.data, w.ctypes.data,
                                 aux.ctypes.data, 16, 1, GEMV_I, GEMV_O, GS) == 1
    n = 400

    def timed(fn, n):
        lib.logan_hip_profile_reset()
        lib.logan_hip_profile_set_on(1)
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        wall = (time.perf_counter() - t0) / n * 1e6
        lib.logan_hip_profile_set_on(0)
        v = [C.c_uint64(0) for _ in range(4)]
        lib.logan_hip_profile_get(*[C.byref(c) for c in v])
        return wall, v[3].value / n / 1e3

    wall, kern = timed(lambda: lib.coli_metal_matmul(C.byref(t), y.ctypes.data, x.ctypes.data,
                                                     w.ctypes.data, aux.ctypes.data, 16, 1,
                                                     GEMV_I, GEMV_O, GS), n)
    lib.logan_hip_tensor_free(t)
    res["gemv_config1"] = dict(us_per_call_wall=round(wall, 2), us_device=round(kern, 2),
                               gbps_device=round(GEMV_BYTES / (kern * 1e-6) / 1e9, 1),
                               calls=n, path="coli_metal_matmul (fmt 16)")
    log(f"drop-in gemv: {wall:.1f} us/call wall, {kern:.2f} us device")
    # ---- config-3 layer, B = 1
    nexp = 64
    g = synth.make_affine(rng, INTER, D, BITS, GS, E=nexp)
    u = synth.make_affine(rng, INTER, D, BITS, GS, E=nexp)
    dn = synth.make_affine(rng, D, INTER, BITS, GS, E=nexp)
    sg, su, sd = (synth.make_affine(rng, INTER, D, BITS, GS), synth.make_affine(rng, INTER, D, BITS, GS),
                  synth.make_affine(rng, D, INTER, BITS, GS))
    se_g = synth.bf16_to_f32(synth.bf16_bits(rng.standard_normal(D).astype(np.float32) * 0.05))

    def desc(t3, e, o, i):
        ww, ss, bb = t3
        if e is not None:
            ww, ss, bb = ww[e], ss[e], bb[e]
        return backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32), ww,
                                           synth.aux_bytes(ss, bb), BITS, GS, False, i, o)

    experts = [[desc(g, e, INTER, D), desc(u, e, INTER, D), desc(dn, e, D, INTER)] for e in range(nexp)]
    shared = [desc(sg, None, INTER, D), desc(su, None, INTER, D), desc(sd, None, D, INTER)]
    xs = [synth.bf16_to_f32(synth.make_x(rng, D)) for _ in range(16)]
    lgs = [synth.bf16_to_f32(synth.make_logits(rng, 1, nexp)[0]) for _ in range(16)]
    out = np.zeros(D, np.float32)

    def layer(i):
        xv, lg = xs[i % 16], lgs[i % 16]
        p = np.exp(lg - lg.max())
        p /= p.sum()
        idx = np.argsort(-p, kind="stable")[:TOPK]
        wts = p[idx] / p[idx].sum()
        pend = backend.moe_route_begin([d for e in idx for d in experts[e]], xv, D, INTER)
        sy = np.zeros(D, np.float32)
        assert backend.shared_expert(shared, xv, sy, D, INTER)
        ys = np.zeros(TOPK * D, np.float32)
        assert backend.moe_route_finish(pend, ys) == 1
        acc = np.zeros(D, np.float32)
        for r in range(TOPK):
            acc += ys[r * D:(r + 1) * D] * wts[r]
        gs_ = 1.0 / (1.0 + np.exp(-float(se_g @ xv)))
        out[:] = acc + sy * np.float32(gs_)

    for i in range(nexp):  # first use uploads every expert's handles
        layer(i)
    nl = 100
    wall, kern = timed(lambda: layer(np.random.randint(16)), nl)
    per_layer_bytes = (TOPK + 1) * PER_EXPERT
    res["moe_b1_config3"] = dict(us_per_layer_wall=round(wall, 1), us_device=round(kern, 1),
                                 gbps_device=round(per_layer_bytes / (kern * 1e-6) / 1e9, 1),
                                 layers=nl, experts_resident=nexp,
                                 path="coli_metal_moe_route_begin + coli_metal_shared_mxfp4 + "
                                      "coli_metal_moe_route_finish, host routing and combine")
    log(f"drop-in moe layer: {wall:.1f} us wall, {kern:.1f} us device")
    for e in experts:
        for d in e:
            d.tensor.free()
    for d in shared:
        d.tensor.free()
    return res


def measured_traffic():
    """HBM bytes per fused-MoE launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy of known
    size), or None when the summary is absent."""
    f = ROOT / "profiles" / "moe_fused_b1_config3_traffic.json"
    if not f.exists():
        return None
    return json.loads(f.read_text()).get("hbm_bytes_per_launch")


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, layer, seconds):
    """The reference's CPU path restated by the oracle (oracle/oracle.c), on
    the host cores of this box, on bounded samples of the same workloads:
    the config-3 MoE token (softmax top-10, 11 expert MLPs, rank-ordered
    combine, shared expert) and the config-1 q4 GEMV, each with 1 thread
    (what the reference runs: logan-qwen4/src/lib.rs:3752-3763, :8759) and
    row-parallel over the host threads (its own row split, :3785-3807).
    Each figure is the median of 5 runs; `seconds` bounds the whole leg."""
    import os

    import numpy as np

    import oracle
    from logan_amd import synth

    def host(b):
        return (b.weights.cpu().numpy(), b.scales.cpu().numpy().view(np.uint16),
                b.biases.cpu().numpy().view(np.uint16))

    gate, up, down = host(layer.gate), host(layer.up), host(layer.down)
    shared = tuple(tuple(a[0] for a in host(b)) for b in (layer.shared_gate, layer.shared_up,
                                                          layer.shared_down))
    se_g = layer.shared_gate_vec.float().cpu().numpy()
    rng = np.random.default_rng(0)
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = nproc
    # the box's share for one GPU is 16 threads (the reference's default is
    # n - 1 of the available threads, lib.rs:3660-3675)
    par = max(1, min(16, avail - 1 if avail > 1 else 1))
    xs = [synth.bf16_to_f32(synth.make_x(rng, D)) for _ in range(4)]
    lgs = [synth.bf16_to_f32(synth.make_logits(rng, 1, E)[0]) for _ in range(4)]
    gw, gsc, gbi = synth.make_affine(rng, GEMV_O, GEMV_I, BITS, GS)
    gx = synth.bf16_to_f32(synth.make_x(rng, GEMV_I))

    def runs(fn, total_s):
        """5 runs sharing about total_s: median seconds per call."""
        t0 = time.perf_counter()
        fn(0)
        once = max(time.perf_counter() - t0, 1e-6)
        n = max(1, int(total_s / 5 / once))
        res = []
        for r in range(5):
            t0 = time.perf_counter()
            for i in range(n):
                fn(i)
            res.append((time.perf_counter() - t0) / n)
        return float(np.median(res)), n

    budget = max(seconds, 5.0) / 2.0  # per thread count, over both workloads
    out = {}
    for name, th in (("1thread", 1), ("parallel", par)):
        moe_s, moe_n = runs(lambda i: oracle.moe_token(xs[i % 4], lgs[i % 4], TOPK, D, INTER, BITS,
                                                       GS, gate, up, down, shared, se_g,
                                                       nthreads=th), budget * 0.8)
        gemv_s, gemv_n = runs(lambda i: oracle.affine_gemv(gx, gw, gsc, gbi, GEMV_O, GEMV_I, BITS,
                                                           GS, nthreads=th), budget * 0.2)
        out[name] = dict(threads=th, moe_us_per_token_layer=round(moe_s * 1e6, 1),
                         moe_gbps=round(LAYER_BYTES_B1 / moe_s / 1e9, 4), moe_calls_per_run=moe_n,
                         gemv_us=round(gemv_s * 1e6, 1),
                         gemv_gbps=round(GEMV_BYTES / gemv_s / 1e9, 4), gemv_calls_per_run=gemv_n)
        log(f"cpu {name} ({th} threads): moe {moe_s * 1e6:.0f} us/token-layer, "
            f"gemv {gemv_s * 1e6:.0f} us")
    one = out["1thread"]
    return dict(value=one["moe_gbps"], unit="GB/s", cores=1, kind="port",
                us_per_token_layer=one["moe_us_per_token_layer"],
                sample=(f"config-3 MoE token (B=1, 4-bit, E=512, top-10 + shared) through the "
                        f"oracle's lo_moe_token, median of 5 runs of {one['moe_calls_per_run']} "
                        f"tokens, 1 thread"),
                row_parallel=out["parallel"], single_thread=one,
                gemv_config1={"1thread_us": one["gemv_us"], "1thread_gbps": one["gemv_gbps"],
                              "parallel_us": out["parallel"]["gemv_us"],
                              "parallel_gbps": out["parallel"]["gemv_gbps"],
                              "parallel_threads": par},
                nproc=nproc, threads_available=avail, cpu_model=cpu_model(), stat="median of 5")


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
    log(f"building {args.layers} resident MoE layers ({args.layers * 0.906:.1f} GB)")
    layers = build_layers(torch, device, synth, args.layers)
    moe = bench_moe(torch, device, synth, args, layers)
    secondary = {}
    legs = set() if args.no_secondary or args.legs == "none" else set(args.legs.split(","))
    if args.no_gemv:
        legs.discard("gemv")
    if legs:
        if "gemv" in legs:
            gemv = bench_gemv(torch, device, synth, args)
            secondary["gemv_q4_config1"] = {
                "shape": "M=1 K=2048 N=4096 4-bit g64", "bytes_per_launch": GEMV_BYTES,
                "us_per_launch": round(gemv["us_per_launch"], 3), "gbps": round(gemv["gbps"], 1),
                "frac_of_peak": round(gemv["gbps"] / PEAK_GBPS, 4), "launches": gemv["launches"],
                "rotation": "64 weight copies (302 MB) > 256 MB MALL"}
        if "dense8" in legs:
            secondary["dense8_config2"] = bench_config2(torch, device, synth, args)
        if "llama" in legs:
            secondary["llama_layer_config2"] = bench_llama(torch, device, synth, args)
        if "moe3" in legs:
            c3 = {}
            for B in (16, 32):
                r = moe_batch_leg(torch, device, synth, layers, B, BITS, PER_EXPERT, None, args.reps,
                                  seed=300 + B)
                log(f"config 3 B={B}: {r['us_per_layer']} us/layer, {r['gbps']} GB/s, "
                    f"U={r['distinct_experts']}")
                c3[f"B{B}"] = r
            secondary["moe_config3"] = c3
        if "stack5" in legs:
            secondary["stack_config5"] = bench_config5(torch, device, synth, args, layers)
        if "moe4" in legs:
            secondary["moe_config4"] = bench_config4(torch, device, synth, args)
        if "router" in legs:
            secondary["moe3_router_on_device"] = bench_router(torch, device, synth, args, layers)
        if "dropin" in legs:
            secondary["dropin"] = bench_dropin(torch, synth, args)
        if "mxfp4" in legs:
            secondary["mxfp4"] = bench_mxfp4(torch, device, args)
        if "loader" in legs:
            secondary["loader"] = bench_loader(torch, args)
        if "cache" in legs:
            secondary["expert_cache"] = bench_cache(torch, device, synth, args, layers)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(torch, layers[0], args.cpu_seconds)
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
    if secondary:
        res["secondary"] = secondary
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
