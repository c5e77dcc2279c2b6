"""Stage timeline of the fused B = 1 routed-MoE launch (`moe_fused_b1_kernel`).

`python logan_amd/build.py --timeline` builds logan_amd/liblogan_hip_timeline.so:
the library with moe_fused.hip compiled under LOGAN_HIP_TIMELINE, whose blocks
record s_memrealtime stamps (100 MHz) of their stages. `python -m
logan_amd.timeline` then runs config-3 layers (B = 1, 4-bit g64, E = 512,
top-10 + one shared expert, D = 2048, inter = 512, `--bits` 4/5/6/8, bf16 logits or
`--f32-logits`; each layer its own seeded
weights, x and router logits) as one HIP graph of `--layers` fused launches,
replays it, reads the stamps of the graph's last two launches and prints, per
stage, the distribution over blocks in microseconds from the first block
start of that launch.

A blocks (gate/up + SwiGLU, one expert slot each): start, route known (the
block's wave 0 has selected its expert and the launch ticket is back), gate/up
weights consumed (wave 0), arrival added (the block's last wave).
B blocks (down + combine, 8 output rows each): start, route known, arrivals
seen, h read, down products formed (these three: the latest wave of the
block), end (outputs stored).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent

E, TOPK, D, INTER, GS = 512, 10, 2048, 512, 64
# grid of the D = 2048 instantiations: 4 gate/up rows per A wave (2 for 8-bit
# codes), 8 waves per block, (k + 1) * inter / (8 * rows) A blocks; 8 output
# rows per B block
N_B = D // 8


def n_a(bits: int) -> int:
    return (TOPK + 1) * INTER // ((2 if bits == 8 else 4) * 8)
A_STAGES = ("start", "route known", "gate/up weights consumed", "arrival added")
B_STAGES = ("start", "route known", "arrivals seen", "h read", "down products", "end")


def _layers(torch, device, synth, n, BITS):
    layers = []
    for l in range(n):
        s = 1000 * l

        def bank(O, I, cnt, seed):
            w, sc, bi = synth.torch_affine(O, I, BITS, GS, E=cnt, seed=seed)
            return device.AffineBank(w, sc, bi, cnt, O, I, BITS, GS)

        g = torch.Generator(device="cuda")
        g.manual_seed(s + 7)
        se_g = (torch.randn(D, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        layers.append(device.MoeLayer(bank(INTER, D, E, s + 1), bank(INTER, D, E, s + 2),
                                      bank(D, INTER, E, s + 3), TOPK, bank(INTER, D, 1, s + 4),
                                      bank(INTER, D, 1, s + 5), bank(D, INTER, 1, s + 6), se_g))
    return layers


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--bits", type=int, default=4, choices=(4, 5, 6, 8))
    ap.add_argument("--f32-logits", action="store_true",
                    help="f32 router logits (64-bit selection keys) instead of bf16")
    args = ap.parse_args(argv)

    from logan_amd import build as b

    if not b.TIMELINE_LIB.exists():
        print(f"{b.TIMELINE_LIB} is missing: run `python logan_amd/build.py --timeline` first",
              file=sys.stderr)
        return 2
    os.environ["LOGAN_HIP_LIB"] = str(b.TIMELINE_LIB)
    import numpy as np
    import torch

    from logan_amd import _lib, device, synth

    L = args.layers
    N_A = n_a(args.bits)
    layers = _layers(torch, device, synth, L, args.bits)
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    xs = torch.randn((L, 1, D), device="cuda", generator=g).to(torch.bfloat16)
    lg = torch.randn((L, 1, E), device="cuda", generator=g)
    if not args.f32_logits:
        lg = lg.to(torch.bfloat16)
    out = torch.empty((L, 1, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")

    def step():
        for l in range(L):
            device.moe_block(layers[l], xs[l], lg[l], out=out[l], workspace=ws)

    step()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        step()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        gr.replay()
        ev0.record(stream)
        for _ in range(args.reps):
            gr.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (args.reps * L)

    fn = _lib.lib().logan_hip_fused_timeline
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    st = np.zeros((2, 1024, 16), dtype=np.uint64)
    if fn(st.ctypes.data, st.nbytes) != 0:
        raise RuntimeError("reading the timeline stamps failed")
    nb = N_A + N_B
    ends = [st[p, N_A:nb, 5].max() for p in range(2)]
    last = int(np.argmax(ends))
    prev = 1 - last
    t = st[last, :nb].astype(np.int64)
    t0 = t[:, 0].min()
    gap = (t0 - int(st[prev, N_A:nb, 5].max())) / 100.0
    kind = "f32" if args.f32_logits else "bf16"
    print(f"config 3 B=1 ({args.bits}-bit, {kind} logits), {L} layers: {us:.2f} us per launch (graph replay, timeline build); "
          f"{N_A} A + {N_B} B blocks")
    print(f"previous launch's last block end -> this launch's first block start: {gap:.2f} us")
    print("| blocks | stage | min | median | p90 | max |")
    print("|---|---|---:|---:|---:|---:|")
    for kind, lo, hi, names in (("A", 0, N_A, A_STAGES), ("B", N_A, nb, B_STAGES)):
        for j, name in enumerate(names):
            v = (t[lo:hi, j] - t0) / 100.0
            print(f"| {kind} | {name} | {v.min():.2f} | {np.median(v):.2f} | "
                  f"{np.percentile(v, 90):.2f} | {v.max():.2f} |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
