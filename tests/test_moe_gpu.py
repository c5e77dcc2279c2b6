"""GPU parity of the router top-k and the routed-MoE block against the oracle.

Bars: routing indices bit-exact (same experts, same rank order, ties to the
lower index); routing weights within 1e-5 relative; MoE f32 output within
max|y-ŷ|/max|ŷ| <= 2e-3 of the oracle (observed ~1e-6); bf16 output ==
RNE(f32 output) bit for bit; B>1 rows identical to B=1 runs of the same
token (grouping does not change any token's arithmetic).
"""
import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32, make_affine, make_logits, make_x

from _util import normwise_rel

pytestmark = pytest.mark.gpu
TOL = 2e-3


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def oracle_route(logits_f32, k):
    probs = oracle.softmax_row(logits_f32)
    idx, val, wsum = oracle.topk(probs, k)
    return idx, (val / np.float32(wsum)).astype(np.float32)


@pytest.mark.parametrize("E,k,B,kind", [(512, 10, 64, "normal"), (512, 10, 32, "zipf"),
                                        (512, 10, 16, "ties"), (100, 7, 5, "normal"),
                                        (32, 32, 3, "normal"), (1024, 32, 4, "normal"),
                                        (512, 1, 8, "ties"), (8, 2, 9, "ties")])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_route_topk_bit_exact(gpu, E, k, B, kind, dtype):
    import torch
    from logan_amd.device import route_topk

    rng = np.random.default_rng(E + k + B)
    lb = make_logits(rng, B, E, zipf_s=1.1 if kind == "zipf" else None)
    lf = bf16_to_f32(lb)
    if kind == "ties":
        for b in range(B):
            order = np.argsort(-lf[b], kind="stable")
            lo, hi = max(0, k - 3), min(E, k + 3)
            lf[b, order[lo:hi]] = lf[b, order[lo]]
            lf[b, order[hi:hi + 4]] = lf[b, order[-1]]
        lb = bf16_bits(lf)
    if dtype == "bf16":
        ld = to_dev(lb.view(np.int16), torch).view(torch.bfloat16)
    else:
        ld = to_dev(lf, torch)
    idx, w = route_topk(ld, k)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    for b in range(B):
        ri, rw = oracle_route(lf[b], k)
        np.testing.assert_array_equal(idx[b], ri)
        np.testing.assert_allclose(w[b], rw, rtol=1e-5, atol=1e-7)


def test_route_rejects_out_of_range_k(gpu):
    import torch
    from logan_amd.device import LoganHipError, route_topk

    lg = torch.zeros((1, 64), device="cuda")
    for k in (0, 33, 65):
        with pytest.raises(LoganHipError):
            route_topk(lg, k)
    with pytest.raises(LoganHipError):
        route_topk(torch.zeros((1, 1025), device="cuda"), 4)


def test_route_negative_zero_and_equal_logits(gpu):
    import torch
    from logan_amd.device import route_topk

    lf = np.zeros((2, 16), np.float32)
    lf[0, ::2] = -0.0
    lf[1] = 1.0
    idx, w = route_topk(to_dev(lf, torch), 4)
    for b in range(2):
        ri, rw = oracle_route(lf[b], 4)
        np.testing.assert_array_equal(idx.cpu().numpy()[b], ri)
        np.testing.assert_allclose(w.cpu().numpy()[b], rw, rtol=1e-6)


class Layer:
    """Seeded MoE layer in the benchmark scheme, host copies + device banks."""

    def __init__(self, torch, E, k, D, inter, bits, gs, shared=True, seed=0, sinter=None,
                 fp16=False):
        from logan_amd.device import AffineBank, MoeLayer

        rng = np.random.default_rng(seed)
        self.E, self.k, self.D, self.inter, self.bits, self.gs = E, k, D, inter, bits, gs
        self.fp16 = fp16
        self.sinter = inter if sinter is None else sinter
        self.gate = make_affine(rng, inter, D, bits, gs, fp16, E=E)
        self.up = make_affine(rng, inter, D, bits, gs, fp16, E=E)
        self.down = make_affine(rng, D, inter, bits, gs, fp16, E=E)

        def bank(t, O, I, n):
            w, sc, bi = t
            return AffineBank(to_dev(w, torch), to_dev(sc.view(np.int16), torch),
                              to_dev(bi.view(np.int16), torch), n, O, I, bits, gs, fp16)

        kw = {}
        self.shared = None
        self.se_g = None
        if shared:
            si = self.sinter
            sg = make_affine(rng, si, D, bits, gs, fp16, E=1)
            su = make_affine(rng, si, D, bits, gs, fp16, E=1)
            sd = make_affine(rng, D, si, bits, gs, fp16, E=1)
            self.shared = tuple(tuple(a[0] for a in t) for t in (sg, su, sd))
            self.se_g_bits = bf16_bits(rng.standard_normal(D).astype(np.float32) * np.float32(0.05))
            self.se_g = bf16_to_f32(self.se_g_bits)
            kw = dict(shared_gate=bank(sg, si, D, 1), shared_up=bank(su, si, D, 1),
                      shared_down=bank(sd, D, si, 1),
                      shared_gate_vec=to_dev(self.se_g_bits.view(np.int16), torch).view(torch.bfloat16))
        self.dev = MoeLayer(bank(self.gate, inter, D, E), bank(self.up, inter, D, E),
                            bank(self.down, D, inter, E), k, **kw)

    def ref(self, xf, lf):
        return oracle.moe_token(xf, lf, self.k, self.D, self.inter, self.bits, self.gs, self.gate,
                                self.up, self.down, self.shared, self.se_g, sinter=self.sinter,
                                fp16=self.fp16)


def run_layer(torch, layer, xb, lb, out_dtype):
    from logan_amd.device import moe_block

    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    lg = to_dev(lb.view(np.int16), torch).view(torch.bfloat16)
    out, idx, w = moe_block(layer.dev, x, lg, return_routing=True, out_dtype=out_dtype)
    return out, idx.cpu().numpy(), w.cpu().numpy()


@pytest.fixture
def fused_mode(request):
    """Force the single-launch B=1 path on or off for one test, restore after."""
    from logan_amd import _lib

    on = getattr(request, "param", 1)
    _lib.lib().logan_hip_set_moe_fused(on)
    yield on
    _lib.lib().logan_hip_set_moe_fused(1)
    assert _lib.lib().logan_hip_moe_sync_errors() == 0


MOE_CASES = [(4, 1, False), (4, 16, False), (4, 40, True), (5, 1, True), (6, 1, True),
             (5, 32, True), (6, 32, True), (8, 4, False), (8, 1, False)]


# B > 1 always takes the multi-launch path, so only B = 1 runs both ways
@pytest.mark.parametrize("fused_mode,bits,B,zipf",
                         [(1, *c) for c in MOE_CASES] + [(0, *c) for c in MOE_CASES if c[1] == 1],
                         indirect=["fused_mode"])
def test_moe_block_matches_oracle(gpu, fused_mode, bits, B, zipf):
    """Configs 3 and 4: E=512, top-10, D=2048, inter=512, g64, shared expert."""
    import torch

    print(f"moe bits={bits} B={B} zipf={zipf} fused={fused_mode}", flush=True)
    layer = Layer(torch, 512, 10, 2048, 512, bits, 64, seed=bits * 10 + B)
    rng = np.random.default_rng(1000 + B)
    xb = make_x(rng, B, 2048)
    lb = make_logits(rng, B, 512, zipf_s=1.1 if zipf else None)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    out16, idx2, _ = run_layer(torch, layer, xb, lb, torch.bfloat16)
    out32 = out32.cpu().numpy()
    out16 = out16.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(idx, idx2)
    np.testing.assert_array_equal(out16, bf16_bits(out32))
    xf, lf = bf16_to_f32(xb), bf16_to_f32(lb)
    for t in range(B):
        ref, ridx, rw = layer.ref(xf[t], lf[t])
        np.testing.assert_array_equal(idx[t], ridx)
        np.testing.assert_allclose(w[t], rw, rtol=1e-5)
        err = normwise_rel(out32[t], ref)
        assert err <= TOL, f"token {t}: {err:.3e}"
        assert err <= 5e-5, f"token {t}: {err:.3e} (expected f32-accumulation level)"


@pytest.mark.parametrize("fused_mode", [0], indirect=True)
def test_moe_batch_rows_equal_single_token_runs(gpu, fused_mode):
    """With the multi-launch path for every B, grouping tokens by expert does
    not change any token's arithmetic: rows of a B=12 run are bit-identical to
    B=1 runs."""
    import torch

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=3)
    rng = np.random.default_rng(4)
    B = 12
    xb = make_x(rng, B, 2048)
    lb = make_logits(rng, B, 512, zipf_s=1.1)
    full, _, _ = run_layer(torch, layer, xb, lb, torch.float32)
    for t in range(B):
        one, _, _ = run_layer(torch, layer, xb[t:t + 1], lb[t:t + 1], torch.float32)
        assert torch.equal(full[t:t + 1], one)


def test_moe_without_shared_expert_and_small_shapes(gpu):
    import torch

    layer = Layer(torch, 16, 4, 256, 128, 4, 32, shared=False, seed=9)
    rng = np.random.default_rng(10)
    B = 5
    xb = make_x(rng, B, 256)
    lb = make_logits(rng, B, 16)
    out, idx, _ = run_layer(torch, layer, xb, lb, torch.float32)
    out = out.cpu().numpy()
    xf, lf = bf16_to_f32(xb), bf16_to_f32(lb)
    for t in range(B):
        ref, ridx, _ = layer.ref(xf[t], lf[t])
        np.testing.assert_array_equal(idx[t], ridx)
        assert normwise_rel(out[t], ref) <= 5e-5


def test_moe_shared_inter_differs(gpu):
    import torch

    layer = Layer(torch, 32, 4, 512, 256, 4, 64, seed=11, sinter=384)
    rng = np.random.default_rng(12)
    xb = make_x(rng, 3, 512)
    lb = make_logits(rng, 3, 32)
    out, idx, _ = run_layer(torch, layer, xb, lb, torch.float32)
    out = out.cpu().numpy()
    for t in range(3):
        ref, ridx, _ = layer.ref(bf16_to_f32(xb[t]), bf16_to_f32(lb[t]))
        np.testing.assert_array_equal(idx[t], ridx)
        assert normwise_rel(out[t], ref) <= 5e-5


def test_moe_deterministic_and_workspace(gpu):
    import torch
    from logan_amd.device import moe_block

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=21)
    rng = np.random.default_rng(22)
    x = to_dev(make_x(rng, 2, 2048).view(np.int16), torch).view(torch.bfloat16)
    lg = to_dev(make_logits(rng, 2, 512).view(np.int16), torch).view(torch.bfloat16)
    ws = torch.empty(layer.dev.workspace_bytes(2), dtype=torch.uint8, device="cuda")
    a = moe_block(layer.dev, x, lg, workspace=ws, out_dtype=torch.float32)
    b = moe_block(layer.dev, x, lg, out_dtype=torch.float32)
    c = moe_block(layer.dev, x, lg, workspace=ws, out_dtype=torch.float32)
    assert torch.equal(a, b) and torch.equal(a, c)


def test_moe_fused_repeated_launches_are_identical(gpu, fused_mode):
    """200 back-to-back single-launch calls (different routes each time, the
    last repeated): counters return to rest, outputs are deterministic."""
    import torch
    from logan_amd import _lib
    from logan_amd.device import moe_block

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=31)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    xs = torch.randn((200, 1, 2048), device="cuda", generator=g).to(torch.bfloat16)
    ls = torch.randn((200, 1, 512), device="cuda", generator=g).to(torch.bfloat16)
    ws = torch.empty(layer.dev.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    out = torch.empty((200, 1, 2048), dtype=torch.float32, device="cuda")
    for i in range(200):
        moe_block(layer.dev, xs[i], ls[i], out=out[i], workspace=ws)
    again = moe_block(layer.dev, xs[199], ls[199], workspace=ws, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert _lib.lib().logan_hip_moe_sync_errors() == 0
    assert torch.equal(again, out[199])
    assert torch.isfinite(out).all()


def test_moe_fused_agrees_with_multi_launch(gpu):
    import torch
    from logan_amd import _lib

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=41)
    rng = np.random.default_rng(42)
    xb = make_x(rng, 1, 2048)
    lb = make_logits(rng, 1, 512)
    try:
        _lib.lib().logan_hip_set_moe_fused(1)
        a, ia, wa = run_layer(torch, layer, xb, lb, torch.float32)
        _lib.lib().logan_hip_set_moe_fused(0)
        b, ib, wb = run_layer(torch, layer, xb, lb, torch.float32)
    finally:
        _lib.lib().logan_hip_set_moe_fused(1)
    np.testing.assert_array_equal(ia, ib)
    np.testing.assert_allclose(wa, wb, rtol=1e-6)
    assert normwise_rel(a.cpu().numpy(), b.cpu().numpy()) < 2e-5
    assert _lib.lib().logan_hip_moe_sync_errors() == 0


@pytest.mark.parametrize("fused_mode", [1], indirect=True)
@pytest.mark.parametrize("E,k,D,inter,sinter,bits,gs,shared,fp16", [
    (16, 4, 256, 128, None, 4, 32, False, False),   # 4 chunks per row, no shared expert
    (32, 4, 512, 256, 384, 4, 64, True, False),     # shared inter wider than routed
    (64, 8, 512, 384, 128, 6, 64, True, False),     # shared inter narrower than routed
    (64, 8, 4096, 256, None, 4, 64, True, False),   # two x chunks per lane (D > 2048)
    (64, 8, 4096, 256, None, 6, 64, True, False),
    (64, 8, 4096, 256, None, 8, 64, True, True),
    (64, 8, 4096, 256, None, 5, 64, True, False),   # 5-bit at D > 2048: multi-launch path
    (64, 6, 1024, 1024, None, 4, 64, True, False),  # 32 chunks per row
    (64, 6, 1024, 1024, 512, 8, 64, True, False),
    (64, 6, 1024, 768, None, 5, 128, True, True),
    (64, 6, 1024, 640, None, 6, 32, True, False),
    (32, 11, 512, 512, None, 6, 64, True, True),    # 12 slots, the most one launch serves
    (1024, 10, 2048, 512, None, 4, 64, True, False),
    (64, 1, 512, 256, None, 4, 64, True, False),    # k = 1: two slots, most B waves own none
    (128, 2, 1024, 256, None, 8, 64, False, False), # k = 2, no shared expert
    (256, 8, 2048, 512, None, 5, 64, True, False),  # E between the 64 and 512 lane blocks
])
def test_moe_fused_shapes(gpu, fused_mode, E, k, D, inter, sinter, bits, gs, shared, fp16):
    """Single-token block over the shapes the one-launch kernel serves (row
    chunks 4..32, shared width above/below the routed one, D up to 4096, 5/6/8
    bit, fp16 sidecars, group sizes 32..128, 1..12 slots) against the oracle."""
    import torch

    print(f"fused shape E={E} k={k} D={D} inter={inter} sinter={sinter} bits={bits} gs={gs}",
          flush=True)
    layer = Layer(torch, E, k, D, inter, bits, gs, shared=shared, seed=E + k + D + bits,
                  sinter=sinter, fp16=fp16)
    rng = np.random.default_rng(D + inter)
    for rep in range(2):
        xb = make_x(rng, 1, D)
        lb = make_logits(rng, 1, E)
        out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
        out16, idx2, _ = run_layer(torch, layer, xb, lb, torch.bfloat16)
        out32 = out32.cpu().numpy()
        np.testing.assert_array_equal(idx, idx2)
        np.testing.assert_array_equal(out16.view(torch.int16).cpu().numpy().view(np.uint16),
                                      bf16_bits(out32))
        ref, ridx, rw = layer.ref(bf16_to_f32(xb[0]), bf16_to_f32(lb[0]))
        np.testing.assert_array_equal(idx[0], ridx)
        np.testing.assert_allclose(w[0], rw, rtol=1e-5)
        err = normwise_rel(out32[0], ref)
        assert err <= 5e-5, f"rep {rep}: {err:.3e}"


@pytest.fixture
def mfma_min_b(request):
    """Set the smallest batch that takes the MFMA path for one test, restore
    the default after."""
    from logan_amd import _lib

    b = getattr(request, "param", 1)
    _lib.lib().logan_hip_set_moe_mfma_min_batch(b)
    yield b
    _lib.lib().logan_hip_set_moe_mfma_min_batch(0)


def _check_tokens(layer, xb, lb, out32, idx, w, tokens):
    xf, lf = bf16_to_f32(xb), bf16_to_f32(lb)
    for t in tokens:
        ref, ridx, rw = layer.ref(xf[t], lf[t])
        np.testing.assert_array_equal(idx[t], ridx)
        np.testing.assert_allclose(w[t], rw, rtol=1e-5)
        err = normwise_rel(out32[t], ref)
        assert err <= 5e-5, f"token {t}: {err:.3e} (expected f32-accumulation level)"


@pytest.mark.parametrize("mfma_min_b", [1], indirect=True)
@pytest.mark.parametrize("bits,B,zipf,shared", [(4, 2, False, True), (4, 16, False, True),
                                                (8, 5, False, True), (4, 40, True, True),
                                                (8, 33, True, False), (5, 40, True, True),
                                                (6, 32, True, True), (5, 3, False, False),
                                                (6, 17, False, True),
                                                (5, 136, True, True),    # 8-wave gate/up blocks
                                                (4, 200, True, True),    # LDS-staged 8-wave blocks
                                                (8, 150, True, True)])
def test_moe_mfma_path_matches_oracle(gpu, mfma_min_b, bits, B, zipf, shared):
    """The token-batch MFMA path (forced for every B) against the oracle:
    routing bit-exact, outputs at f32-accumulation level; Zipf routes put
    more than 16 tokens on the popular experts (several tiles per expert)."""
    import torch

    print(f"moe mfma bits={bits} B={B} zipf={zipf} shared={shared}", flush=True)
    layer = Layer(torch, 512, 10, 2048, 512, bits, 64, seed=bits * 7 + B, shared=shared)
    rng = np.random.default_rng(2000 + B)
    xb = make_x(rng, B, 2048)
    lb = make_logits(rng, B, 512, zipf_s=1.1 if zipf else None)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    out16, idx2, _ = run_layer(torch, layer, xb, lb, torch.bfloat16)
    out32 = out32.cpu().numpy()
    np.testing.assert_array_equal(idx, idx2)
    np.testing.assert_array_equal(out16.view(torch.int16).cpu().numpy().view(np.uint16),
                                  bf16_bits(out32))
    if zipf:
        assert np.bincount(idx.reshape(-1)).max() > 16
    _check_tokens(layer, xb, lb, out32, idx, w, range(B))


@pytest.mark.parametrize("mfma_min_b", [1], indirect=True)
@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_moe_mfma_fp16_sidecars(gpu, mfma_min_b, bits):
    """fp16 scale/bias sidecars through the MFMA path (both passes)."""
    import torch

    layer = Layer(torch, 128, 8, 1024, 256, bits, 64, seed=61 + bits, fp16=True)
    rng = np.random.default_rng(62)
    B = 20
    xb = make_x(rng, B, 1024)
    lb = make_logits(rng, B, 128)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    _check_tokens(layer, xb, lb, out32.cpu().numpy(), idx, w, range(B))


@pytest.mark.parametrize("mfma_min_b", [1], indirect=True)
@pytest.mark.parametrize("bits,fp16,D,sinter", [(4, True, 2048, 512), (8, True, 1024, 384),
                                                 (4, False, 1024, 384), (8, False, 2048, 256),
                                                 (4, False, 768, 256)])
def test_moe_mfma_large_batch_staged_weights(gpu, mfma_min_b, bits, fp16, D, sinter):
    """Batches above 128 tokens take the gate/up and down blocks whose 4- and
    8-bit weights are staged in LDS: fp16 and bf16 sidecars, D = 1024 (one
    x chunk shorter than the LDS tile), 2048, and 768 (down blocks of 512
    rows running past D); shared experts whose down K is one, two or three
    batches, or (4-bit, K = 384) not a whole number of them (the register
    down blocks); every 7th token against the oracle."""
    import torch

    print(f"moe mfma staged bits={bits} fp16={fp16} D={D} sinter={sinter}", flush=True)
    layer = Layer(torch, 256, 8, D, 512, bits, 64, seed=71 + bits + D, fp16=fp16, sinter=sinter)
    rng = np.random.default_rng(72 + D)
    B = 160
    xb = make_x(rng, B, D)
    lb = make_logits(rng, B, 256, zipf_s=1.1)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    _check_tokens(layer, xb, lb, out32.cpu().numpy(), idx, w, range(0, B, 7))


@pytest.mark.parametrize("mfma_min_b", [1], indirect=True)
def test_moe_mfma_shapes_and_group_sizes(gpu, mfma_min_b):
    """Smaller shapes through the MFMA path: D = 512 (one LDS chunk), inter =
    256, a shared expert of 384 rows, group size 128."""
    import torch

    layer = Layer(torch, 64, 6, 512, 256, 4, 128, seed=31, sinter=384)
    rng = np.random.default_rng(32)
    B = 24
    xb = make_x(rng, B, 512)
    lb = make_logits(rng, B, 64, zipf_s=1.1)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    _check_tokens(layer, xb, lb, out32.cpu().numpy(), idx, w, range(B))


def test_moe_prefill_chunk_sampled(gpu):
    """A prefill-sized batch (B = 512, the config-5 chunk) with the default
    threshold (MFMA path), checked against the oracle on a sample of tokens,
    and against the per-token path on every token."""
    import torch
    from logan_amd import _lib

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=41)
    rng = np.random.default_rng(42)
    B = 512
    xb = make_x(rng, B, 2048)
    lb = make_logits(rng, B, 512)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    out32 = out32.cpu().numpy()
    _check_tokens(layer, xb, lb, out32, idx, w, range(0, B, 37))
    _lib.lib().logan_hip_set_moe_mfma_min_batch(1 << 20)
    try:
        out_d, idx_d, _ = run_layer(torch, layer, xb, lb, torch.float32)
    finally:
        _lib.lib().logan_hip_set_moe_mfma_min_batch(0)
    np.testing.assert_array_equal(idx, idx_d)
    out_d = out_d.cpu().numpy()
    for t in range(B):
        assert normwise_rel(out32[t], out_d[t]) <= 5e-5


@pytest.mark.parametrize("bits,fp16,D,sinter", [(4, True, 2048, 384), (8, False, 1024, 256),
                                                 (4, False, 768, 512)])
def test_moe_prefill_whole_tile_blocks(gpu, bits, fp16, D, sinter):
    """B = 512 over E = 256, top-8: enough tiles that the LDS-staged gate/up
    and down launches give the first tiles whole-tile blocks and the last
    units one-group / 512-row blocks. Shared experts narrower than the routed
    ones (fewer row groups and a shorter down K in their whole-tile blocks),
    8-bit codes, fp16 sidecars, and D = 768 (down blocks running past D); a
    sample of tokens against the oracle and every token against the
    per-token path."""
    import torch
    from logan_amd import _lib

    print(f"moe whole-tile blocks bits={bits} fp16={fp16} D={D} sinter={sinter}", flush=True)
    layer = Layer(torch, 256, 8, D, 512, bits, 64, seed=91 + bits + D, fp16=fp16, sinter=sinter)
    rng = np.random.default_rng(92 + D)
    B = 512
    xb = make_x(rng, B, D)
    lb = make_logits(rng, B, 256)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    out32 = out32.cpu().numpy()
    _check_tokens(layer, xb, lb, out32, idx, w, range(0, B, 53))
    _lib.lib().logan_hip_set_moe_mfma_min_batch(1 << 20)
    try:
        out_d, idx_d, _ = run_layer(torch, layer, xb, lb, torch.float32)
    finally:
        _lib.lib().logan_hip_set_moe_mfma_min_batch(0)
    np.testing.assert_array_equal(idx, idx_d)
    out_d = out_d.cpu().numpy()
    for t in range(B):
        assert normwise_rel(out32[t], out_d[t]) <= 5e-5


@pytest.mark.parametrize("mfma_min_b", [1 << 20], indirect=True)
def test_moe_large_batch_per_token_passes(gpu, mfma_min_b):
    """With the MFMA path off, B = 100 runs the per-token path in passes of
    64 tokens; every third token against the oracle."""
    import torch

    layer = Layer(torch, 512, 10, 2048, 512, 5, 64, seed=51)
    rng = np.random.default_rng(52)
    B = 100
    xb = make_x(rng, B, 2048)
    lb = make_logits(rng, B, 512, zipf_s=1.1)
    out32, idx, w = run_layer(torch, layer, xb, lb, torch.float32)
    _check_tokens(layer, xb, lb, out32.cpu().numpy(), idx, w, range(0, B, 3))


def test_moe_fused_after_other_paths_on_one_workspace(gpu, fused_mode):
    """The single-launch B=1 path's tagged h pairs must never be confused with
    what else a workspace holds: the workspace starts filled with small odd
    integers (what a stale tag of an early launch looks like), then takes a
    per-token (B=16) and an MFMA (B=64) call, then B=1 calls; every result
    against the oracle."""
    import torch
    from logan_amd import _lib
    from logan_amd.device import moe_block

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=41)
    rng = np.random.default_rng(42)
    ws = torch.arange(1, 2 * (layer.dev.workspace_bytes(64) // 4) + 1, 2, dtype=torch.int32,
                      device="cuda")[: layer.dev.workspace_bytes(64) // 4].contiguous()
    ws8 = ws.view(torch.uint8)
    for B in (16, 64, 1, 1, 1):
        xb = make_x(rng, B, 2048)
        lb = make_logits(rng, B, 512)
        x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
        lg = to_dev(lb.view(np.int16), torch).view(torch.bfloat16)
        out, idx, _ = moe_block(layer.dev, x, lg, workspace=ws8, return_routing=True,
                                out_dtype=torch.float32)
        out, idx = out.cpu().numpy(), idx.cpu().numpy()
        xf, lf = bf16_to_f32(xb), bf16_to_f32(lb)
        for t in range(B):
            ref, ridx, _ = layer.ref(xf[t], lf[t])
            np.testing.assert_array_equal(idx[t], ridx)
            assert normwise_rel(out[t], ref) <= 5e-5, f"B={B} token {t}"
    assert _lib.lib().logan_hip_moe_sync_errors() == 0


def test_moe_fused_launches_on_two_streams(gpu, fused_mode):
    """Single-launch B=1 calls alternating between two streams with no
    synchronisation in between: the library orders them (the launches share
    device-scope counters), every output against a single-stream run."""
    import torch
    from logan_amd import _lib
    from logan_amd.device import moe_block

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=43)
    rng = np.random.default_rng(44)
    n = 12
    xs = [to_dev(make_x(rng, 1, 2048).view(np.int16), torch).view(torch.bfloat16) for _ in range(n)]
    ls = [to_dev(make_logits(rng, 1, 512).view(np.int16), torch).view(torch.bfloat16) for _ in range(n)]
    want = [moe_block(layer.dev, xs[i], ls[i], out_dtype=torch.float32) for i in range(n)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    wss = [torch.empty(layer.dev.workspace_bytes(1), dtype=torch.uint8, device="cuda")
           for _ in range(2)]
    outs = [torch.empty((1, 2048), dtype=torch.float32, device="cuda") for _ in range(n)]
    for i in range(n):
        s = s1 if i % 2 == 0 else s2
        with torch.cuda.stream(s):
            moe_block(layer.dev, xs[i], ls[i], out=outs[i], workspace=wss[i % 2], stream=s)
    torch.cuda.synchronize()
    for i in range(n):
        assert torch.equal(outs[i], want[i]), i
    assert _lib.lib().logan_hip_moe_sync_errors() == 0


@pytest.mark.parametrize("fused_mode,B,rbits,spread",
                         [(1, 1, 8, 0.04), (0, 1, 8, 0.04), (1, 16, 8, 0.04), (1, 64, 4, 0.6),
                          (1, 1, 4, 0.6), (1, 1, 8, 8.0), (1, 16, 8, 8.0)],
                         indirect=["fused_mode"])
def test_moe_block_with_router_on_device(gpu, fused_mode, B, rbits, spread):
    """The router product on device (logan-qwen4/src/lib.rs:7990-7991) feeding
    the block's f32-logit routing: the device logits against the oracle's
    GEMV; the selection on those very logits bit-exact against the oracle's
    softmax + top-k; the output against the oracle's MoE token on them.
    `spread` scales the router: logits near N(0, 1) (the fast selection) or
    in the hundreds (exps below the top one underflow: the recomputed
    reference selection)."""
    import torch
    from logan_amd.device import AffineMatrix, moe_block_routed

    print(f"moe router B={B} router bits={rbits} spread={spread} fused={fused_mode}", flush=True)
    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=61 + B)
    rng = np.random.default_rng(62 + B)
    rw, rsc, rbi = make_affine(rng, 512, 2048, rbits, 64)
    rsc = bf16_bits(bf16_to_f32(rsc) * np.float32(spread))
    rbi = bf16_bits(bf16_to_f32(rsc) * np.float32(-(2 ** (rbits - 1))))
    router = AffineMatrix(to_dev(rw, torch), to_dev(rsc.view(np.int16), torch),
                          to_dev(rbi.view(np.int16), torch), 512, 2048, rbits, 64)
    xb = make_x(rng, B, 2048)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    out, logits, idx, w = moe_block_routed(layer.dev, router, x, return_routing=True,
                                           out_dtype=torch.float32)
    out, logits, idx = out.cpu().numpy(), logits.cpu().numpy(), idx.cpu().numpy()
    xf = bf16_to_f32(xb)
    for t in range(B):
        lref = oracle.affine_gemv(xf[t], rw, rsc, rbi, 512, 2048, rbits, 64)
        assert normwise_rel(logits[t], lref) <= 2e-5
        ref, ridx, _ = layer.ref(xf[t], logits[t])
        np.testing.assert_array_equal(idx[t], ridx)
        assert normwise_rel(out[t], ref) <= 5e-5
