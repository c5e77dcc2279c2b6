"""GPU parity of the affine GEMV paths against the CPU oracle.

Bars: dequantised weights bit-exact; f32 outputs within max|y-ŷ|/max|ŷ| <=
2e-3 of the oracle's fp32 GEMV (observed values are ~1e-6); bf16 outputs
within 1 bf16 ulp of RNE(oracle). The host drop-in path uses the reference
tests' own generators and tolerances (logan-metal/src/lib.rs:1310-1378:
max(2e-3, 2e-4|ref|) per element; logan-qwen4/src/lib.rs:17104-17177: 2e-5
normwise).
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from logan_amd.synth import aux_bytes, bf16_bits, bf16_to_f32, make_affine, make_x

from _util import bf16_ulp_ok, normwise_rel, pack_codes

pytestmark = pytest.mark.gpu
TOL = 2e-3
GOLDEN = json.loads((Path(__file__).parent / "golden" / "kat_vectors.json").read_text())


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16=False):
    from logan_amd.device import AffineMatrix

    return AffineMatrix(to_dev(w, torch), to_dev(sc.view(np.int16), torch),
                        to_dev(bi.view(np.int16), torch), O, I, bits, gs, fp16)


@pytest.mark.parametrize("bits,gs,fp16", [(4, 64, False), (5, 64, False), (6, 64, False),
                                          (8, 64, False), (4, 32, True), (5, 128, False),
                                          (6, 128, True), (8, 32, False)])
def test_dequant_bit_exact(gpu, bits, gs, fp16):
    import torch
    from logan_amd.device import affine_dequant

    rng = np.random.default_rng(bits * 100 + gs)
    O, I = 37, 512
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16)
    got = affine_dequant(m).cpu().numpy()
    want = oracle.affine_dequant(w, sc, bi, O, I, bits, gs, fp16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


SHAPES = [
    # (O, I, bits, gs): config 1, the expert shapes of configs 3-4, odd rows, long K
    (4096, 2048, 4, 64),
    (512, 2048, 4, 64), (2048, 512, 4, 64),
    (512, 2048, 5, 64), (2048, 512, 5, 64),
    (512, 2048, 6, 64), (2048, 512, 6, 64),
    (1000, 4096, 8, 64), (333, 1024, 8, 128), (77, 256, 4, 32), (130, 8192, 4, 64),
    (96, 14336, 8, 64), (64, 12288, 5, 128), (40, 1536, 6, 32),
]


@pytest.mark.parametrize("O,I,bits,gs", SHAPES)
@pytest.mark.parametrize("M", [1, 3, 8, 17])
def test_gemv_bf16_matches_oracle(gpu, O, I, bits, gs, M):
    import torch
    from logan_amd.device import affine_gemv

    print(f"gemv O={O} I={I} bits={bits} gs={gs} M={M}", flush=True)
    rng = np.random.default_rng(O * 7 + I + bits + M)
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    xb = make_x(rng, M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    xd = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y32 = affine_gemv(m, xd, out_dtype=torch.float32).cpu().numpy()
    y16 = affine_gemv(m, xd, out_dtype=torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    xf = bf16_to_f32(xb)
    # the bf16 output is the RNE of the same f32 accumulator
    np.testing.assert_array_equal(y16, bf16_bits(y32))
    for r in range(M):
        ref = oracle.affine_gemv(xf[r], w, sc, bi, O, I, bits, gs)
        err = normwise_rel(y32[r], ref)
        assert err <= TOL, f"row {r}: normwise {err:.3e}"
        assert err <= 2e-5, f"row {r}: normwise {err:.3e} (expected f32-accumulation level)"
        # away from cancellation the bf16 output is within 1 ulp of RNE(oracle)
        big = np.abs(ref) > 1e-2 * np.abs(ref).max()
        assert bf16_ulp_ok(y16[r][big], ref[big], 1)


# (O, I, bits, gs, fp16): the shapes that take the K-split-across-waves kernel
# at 3..8 tokens (at least 4096 rows, I / 512 with a divisor in [4, 8]; M = 16
# takes the K split across blocks): config 2's q/k/v, o and down products,
# odd wave counts (5, 6, 7), ragged rows, groups of 128, fp16 sidecars
KWAVE_SHAPES = [
    (6144, 4096, 8, 64, False), (4096, 4096, 8, 64, False), (4096, 14336, 8, 64, False),
    (4100, 2560, 5, 64, False), (4111, 3072, 6, 128, False), (4096, 3584, 4, 64, True),
    (5000, 4096, 4, 128, False),
]


@pytest.mark.parametrize("O,I,bits,gs,fp16", KWAVE_SHAPES)
@pytest.mark.parametrize("M", [3, 4, 5, 8, 16])
def test_gemv_kwave_matches_oracle(gpu, O, I, bits, gs, fp16, M):
    import torch
    from logan_amd.device import affine_gemv

    print(f"kwave O={O} I={I} bits={bits} gs={gs} fp16={fp16} M={M}", flush=True)
    rng = np.random.default_rng(O + I * 3 + bits * 11 + M)
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16)
    xb = make_x(rng, M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16)
    xd = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y32 = affine_gemv(m, xd, out_dtype=torch.float32).cpu().numpy()
    y16 = affine_gemv(m, xd, out_dtype=torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(y16, bf16_bits(y32))
    xf = bf16_to_f32(xb)
    for r in range(M):
        ref = oracle.affine_gemv(xf[r], w, sc, bi, O, I, bits, gs, fp16=fp16)
        err = normwise_rel(y32[r], ref)
        assert err <= 2e-5, f"row {r}: normwise {err:.3e}"


def test_gemv_fp16_sidecar(gpu):
    import torch
    from logan_amd.device import affine_gemv

    rng = np.random.default_rng(5)
    O, I, bits, gs = 300, 2048, 4, 64
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16=True)
    xb = make_x(rng, 1, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs, True)
    y = affine_gemv(m, to_dev(xb.view(np.int16), torch).view(torch.bfloat16),
                    out_dtype=torch.float32).cpu().numpy()[0]
    ref = oracle.affine_gemv(bf16_to_f32(xb[0]), w, sc, bi, O, I, bits, gs, fp16=True)
    assert normwise_rel(y, ref) <= 1e-4


def test_gemv_is_deterministic(gpu):
    import torch
    from logan_amd.device import affine_gemv

    rng = np.random.default_rng(6)
    O, I = 4096, 2048
    w, sc, bi = make_affine(rng, O, I, 4, 64)
    m = dev_matrix(torch, w, sc, bi, O, I, 4, 64)
    x = to_dev(make_x(rng, 1, I).view(np.int16), torch).view(torch.bfloat16)
    a = affine_gemv(m, x, out_dtype=torch.float32)
    b = affine_gemv(m, x, out_dtype=torch.float32)
    assert torch.equal(a, b)


@pytest.mark.parametrize("M,bits", [(4, 8), (17, 4)])
def test_gemv_splitk_repeats_and_graph_replays(gpu, M, bits):
    """The K-split product's last-arriving block sums the partials and sets
    its row block's counter back to zero: back-to-back calls and replays of a
    captured graph (eager calls in between) all give the same bits, and the
    oracle's values."""
    import torch
    from logan_amd.device import affine_gemv

    O, I, gs = 4096 + 37, 4096, 64
    print(f"splitk repeats O={O} I={I} bits={bits} M={M}", flush=True)
    rng = np.random.default_rng(11 + M)
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    xb = make_x(rng, M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    xd = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    ref0 = affine_gemv(m, xd, out_dtype=torch.float32)
    for _ in range(4):
        assert torch.equal(affine_gemv(m, xd, out_dtype=torch.float32), ref0)
    xf = bf16_to_f32(xb)
    y = ref0.cpu().numpy()
    for r in range(M):
        assert normwise_rel(y[r], oracle.affine_gemv(xf[r], w, sc, bi, O, I, bits, gs)) <= 2e-5
    out = torch.empty_like(ref0)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        out.copy_(affine_gemv(m, xd, out_dtype=torch.float32))
    for _ in range(3):
        out.zero_()
        with torch.cuda.stream(stream):
            gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref0)
        assert torch.equal(affine_gemv(m, xd, out_dtype=torch.float32), ref0)
        torch.cuda.synchronize()
    del gr


def test_gemv_linearity(gpu):
    """W(x1) + W(x2) == W(x1 + x2) up to rounding (size-independent check at
    the config-1 shape)."""
    import torch
    from logan_amd.device import affine_gemv

    rng = np.random.default_rng(8)
    O, I = 4096, 2048
    w, sc, bi = make_affine(rng, O, I, 4, 64)
    m = dev_matrix(torch, w, sc, bi, O, I, 4, 64)
    x1 = torch.randn(1, I, device="cuda").to(torch.bfloat16)
    x2 = torch.randn(1, I, device="cuda").to(torch.bfloat16)
    s = (x1.float() + x2.float()).to(torch.bfloat16)
    # x1 + x2 is exact in bf16 only where no rounding happens; compare in f32
    y1 = affine_gemv(m, x1, out_dtype=torch.float32)
    y2 = affine_gemv(m, x2, out_dtype=torch.float32)
    ys = affine_gemv(m, s, out_dtype=torch.float32)
    exact = ((x1.float() + x2.float()) == s.float()).all().item()
    err = (y1 + y2 - ys).abs().max().item() / ys.abs().max().item()
    assert err < (1e-5 if exact else 2e-2)


@pytest.mark.parametrize("bits,gs", [(4, 64), (5, 128), (8, 64), (6, 32)])
def test_gemv_f32_generic_matches_oracle(gpu, bits, gs):
    import torch
    from logan_amd.device import affine_gemv_f32

    rng = np.random.default_rng(bits + gs)
    O, I, M = 257, 1024, 2
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    x = rng.standard_normal((M, I)).astype(np.float32)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    y = affine_gemv_f32(m, to_dev(x, torch)).cpu().numpy()
    for r in range(M):
        assert normwise_rel(y[r], oracle.affine_gemv(x[r], w, sc, bi, O, I, bits, gs)) < 2e-5


def test_gemv_rejects_bad_geometry(gpu):
    import torch
    from logan_amd.device import AffineMatrix, LoganHipError, affine_gemv

    w = torch.zeros((4, 48), dtype=torch.uint8, device="cuda")
    sc = torch.zeros((4, 3), dtype=torch.int16, device="cuda")
    x = torch.zeros((1, 96), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(LoganHipError):
        affine_gemv(AffineMatrix(w, sc, sc, 4, 96, 4, 48), x)  # group 48 not a multiple of 32


# ------------------------------------------------------------ host drop-in path

@pytest.mark.parametrize("bits,gs", [(4, 64), (5, 128), (6, 64), (8, 128)])
def test_host_matmul_reference_generator(gpu, bits, gs):
    """logan-metal/src/lib.rs:1310-1378 through hip_matmul_mlx_affine."""
    from logan_amd import backend

    O, I = 3, 128
    mask = (1 << bits) - 1
    codes = np.array([[(r * 17 + c * 7 + 3) & mask for c in range(I)] for r in range(O)])
    w = pack_codes(codes, bits)
    g = I // gs
    sc = bf16_bits(np.array([[0.125 * (r + q + 1) for q in range(g)] for r in range(O)], np.float32))
    bi = bf16_bits(np.array([[-0.25 + 0.0625 * (r + q) for q in range(g)] for r in range(O)], np.float32))
    x = np.array([((i % 11) - 5) * 0.125 for i in range(I)], np.float32)
    y = np.zeros(O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul_mlx_affine(t, y, x, w, aux_bytes(sc, bi), bits, gs, False, I, O)
    ref = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs)
    assert np.all(np.abs(y - ref) <= np.maximum(2e-3, 2e-4 * np.abs(ref)))
    # second call reuses the handle
    h = t.handle
    y2 = np.zeros(O, np.float32)
    assert backend.hip_matmul_mlx_affine(t, y2, x, w, aux_bytes(sc, bi), bits, gs, False, I, O)
    assert t.handle == h and np.array_equal(y, y2)
    assert t.nbytes() == w.size + 2 * sc.size * 2
    t.free()


@pytest.mark.parametrize("bits,gs", [(4, 64), (5, 128), (6, 64), (8, 128)])
def test_host_matmul_cuda_twin_generator(gpu, bits, gs):
    """logan-qwen4/src/lib.rs:17104-17177 (the CUDA twin's test): normwise
    max_rel < 2e-5 against matmul_mlx_affine_storage."""
    from logan_amd import backend

    O, I = 7, 128
    x = (np.sin(np.arange(I, dtype=np.float32) * np.float32(0.03125)) * np.float32(0.5)).astype(np.float32)
    mask = (1 << bits) - 1
    codes = np.array([[(r * 11 + c * 7 + 3) & mask for c in range(I)] for r in range(O)])
    w = pack_codes(codes, bits)
    n = O * (I // gs)
    sc = bf16_bits(np.array([0.03125 + (q % 3) * 0.015625 for q in range(n)], np.float32))
    bi = bf16_bits(np.array([-0.125 + (q % 5) * 0.03125 for q in range(n)], np.float32))
    want = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs, nthreads=1)
    t = backend.Tensor()
    for _ in range(2):
        got = np.zeros(O, np.float32)
        assert backend.hip_matmul_mlx_affine(t, got, x, w, aux_bytes(sc, bi), bits, gs, False, I, O)
        assert normwise_rel(got, want) < 2e-5
    t.free()


@pytest.mark.parametrize("case", GOLDEN["gemv"], ids=lambda c: f"b{c['bits']}")
def test_host_matmul_reference_closed_forms(gpu, case):
    from logan_amd import backend

    O, I, bits, gs = case["O"], case["I"], case["bits"], case["group_size"]
    w = np.full((O, I * bits // 8), case["byte"], np.uint8)
    sc = bf16_bits(np.full(O * (I // gs), case["scale"], np.float32))
    bi = bf16_bits(np.full(O * (I // gs), case["bias"], np.float32))
    y = np.zeros(O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul_mlx_affine(t, y, np.full(I, case["x"], np.float32), w,
                                         aux_bytes(sc, bi), bits, gs, False, I, O)
    assert np.all(y == case["expected"])
    t.free()


def test_host_spark_fmt15(gpu):
    """fmt 15 (logan-spark/src/lib.rs:332-344 calls metal_matmul with fmt 15
    then rounds to bf16): equals lo_spark_affine8_gemv after RNE."""
    from logan_amd import backend

    c = GOLDEN["spark_affine8"]
    rng = np.random.default_rng(15)
    O, I = 96, 512
    w, sc, bi = make_affine(rng, O, I, 8, 64)
    aux = aux_bytes(sc, bi)
    x = bf16_to_f32(make_x(rng, I))
    y = np.zeros(O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul(t, y, x, w, aux, 15, I, O)
    yr = bf16_to_f32(bf16_bits(y))
    ref = oracle.spark_affine8_gemv(x, w, aux, O, I)
    assert normwise_rel(yr, ref) < 1e-2 and bf16_ulp_ok(bf16_bits(y), ref, 1)
    t.free()
    # the reference's own closed form
    O, I = c["O"], c["I"]
    aux = np.concatenate([bf16_bits(np.full(O, 1.0, np.float32)),
                          bf16_bits(np.full(O, 0.0, np.float32))])
    y = np.zeros(O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul(t, y, np.ones(I, np.float32), np.full(O * I, 2, np.uint8), aux, 15, I, O)
    assert np.all(y == c["expected"])
    t.free()


def test_host_multi_mixed_formats(gpu):
    """logan-qwen4/src/lib.rs:17015-17053: mixed 5-bit/g128 and 6-bit/g64
    zero-code descriptors with scale = bias = 1 in one submission -> 128;
    plus a private-activation descriptor."""
    from logan_amd import backend

    I = 128

    def desc(bits, gs, o, x=None):
        sc = bf16_bits(np.ones(o * (I // gs), np.float32))
        return backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(o, np.float32),
                                           np.zeros(o * I * bits // 8, np.uint8),
                                           aux_bytes(sc, sc), bits, gs, False, I, o, x)

    d5, d6 = desc(5, 128, 2), desc(6, 64, 3)
    d8 = desc(8, 64, 4, x=np.full(I, 2.0, np.float32))
    backend.dense_profile_start()
    assert backend.hip_matmul_mlx_affine_multi(np.ones(I, np.float32), [d5, d6, d8])
    _, _, _, kernel_ns = backend.dense_profile_stop()
    assert kernel_ns > 0
    assert np.all(d5.y == 128.0) and np.all(d6.y == 128.0) and np.all(d8.y == 256.0)
    for d in (d5, d6, d8):
        assert d.tensor.handle
        d.tensor.free()


def test_host_multi_declines_bad_descriptors(gpu):
    from logan_amd import backend

    I = 128
    sc = bf16_bits(np.ones(2, np.float32))
    bad = backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(1, np.float32),
                                      np.zeros(64, np.uint8), aux_bytes(sc, sc), 4, 48, False,
                                      I, 1)  # 128 % 48 != 0
    assert not backend.hip_matmul_mlx_affine_multi(np.ones(I, np.float32), [bad])
    assert bad.tensor.handle == 0
    assert not backend.hip_matmul_mlx_affine_multi(np.ones(I, np.float32), [])


def _expert_ref(x, g, u, d, D, M, bits, gs):
    gv = oracle.affine_gemv(x, *g, M, D, bits, gs)
    uv = oracle.affine_gemv(x, *u, M, D, bits, gs)
    h = np.array([oracle.lib().lo_silu(float(a)) for a in gv], np.float32) * uv
    return oracle.affine_gemv(h, *d, D, M, bits, gs)


@pytest.mark.parametrize("bits,K", [(4, 10), (5, 4), (6, 3), (8, 2)])
def test_host_route_island(gpu, bits, K):
    """moe_route_begin/finish: K expert outputs, expert-major, against the
    oracle's per-expert SwiGLU MLP."""
    from logan_amd import backend

    rng = np.random.default_rng(bits * 31 + K)
    D, M, gs = 2048, 512, 64
    x = bf16_to_f32(make_x(rng, D))
    descs, mats = [], []
    for _ in range(K):
        g = make_affine(rng, M, D, bits, gs)
        u = make_affine(rng, M, D, bits, gs)
        d = make_affine(rng, D, M, bits, gs)
        mats.append((g, u, d))
        for (w, sc, bi), (o, i) in ((g, (M, D)), (u, (M, D)), (d, (D, M))):
            descs.append(backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32), w,
                                                     aux_bytes(sc, bi), bits, gs, False, i, o))
    pending = backend.moe_route_begin(descs, x, D, M)
    assert pending is not None
    out = np.zeros(K * D, np.float32)
    assert backend.moe_route_finish(pending, out) == 1
    for e, (g, u, d) in enumerate(mats):
        ref = _expert_ref(x, g, u, d, D, M, bits, gs)
        assert normwise_rel(out[e * D:(e + 1) * D], ref) < 1e-4
    # a second route reuses every handle; discard path retires cleanly
    p2 = backend.moe_route_begin(descs, x, D, M)
    p2.close()
    for dsc in descs:
        dsc.tensor.free()


def test_host_route_declines_bad_shapes(gpu):
    from logan_amd import backend

    D, M = 128, 64
    sc = bf16_bits(np.ones(M * 2, np.float32))
    g = backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32),
                                    np.zeros(M * D // 2, np.uint8), aux_bytes(sc, sc), 4, 64,
                                    False, D, M)
    # down with the wrong orientation
    bad_down = backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32),
                                           np.zeros(M * D // 2, np.uint8), aux_bytes(sc, sc), 4,
                                           64, False, D, M)
    assert backend.moe_route_begin([g, g, bad_down], np.ones(D, np.float32), D, M) is None
    assert backend.moe_route_begin([g, g], np.ones(D, np.float32), D, M) is None


def test_host_shared_expert(gpu):
    from logan_amd import backend

    rng = np.random.default_rng(77)
    D, M, bits, gs = 2048, 512, 4, 64
    g, u, d = make_affine(rng, M, D, bits, gs), make_affine(rng, M, D, bits, gs), make_affine(rng, D, M, bits, gs)
    x = bf16_to_f32(make_x(rng, D))
    descs = [backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32), w,
                                         aux_bytes(sc, bi), bits, gs, False, i, o)
             for (w, sc, bi), (o, i) in ((g, (M, D)), (u, (M, D)), (d, (D, M)))]
    out = np.zeros(D, np.float32)
    assert backend.shared_expert(descs, x, out, D, M) is True
    assert normwise_rel(out, _expert_ref(x, g, u, d, D, M, bits, gs)) < 1e-4
    for dsc in descs:
        dsc.tensor.free()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 17])
@pytest.mark.parametrize("shapes", [[(8192, 2048), (512, 2048), (512, 2048)],
                                    [(12288, 2048), (64, 2048)],
                                    [(77, 1024), (300, 1024), (64, 1024), (1000, 1024), (5, 1024),
                                     (128, 1024), (256, 1024), (33, 1024)]],
                         ids=["qkv", "qkvz_ba", "eight"])
def test_gemv_multi_equals_single_launches(gpu, shapes, M, bits):
    """Matrices sharing x in one launch (3..32 tokens: one K-split launch and
    one reduce for all of them): every output bit-identical to its own
    affine_gemv launch, the first against the oracle."""
    import torch
    from logan_amd.device import affine_gemv, affine_gemv_multi

    print(f"multi shapes={len(shapes)} M={M} bits={bits}", flush=True)
    rng = np.random.default_rng(len(shapes) * 10 + M + bits)
    I = shapes[0][1]
    host, mats = [], []
    for O, _ in shapes:
        w, sc, bi = make_affine(rng, O, I, bits, 64)
        host.append((w, sc, bi))
        mats.append(dev_matrix(torch, w, sc, bi, O, I, bits, 64))
    xb = make_x(rng, M, I)
    xd = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    outs = affine_gemv_multi(mats, xd, out_dtype=torch.float32)
    for m, o in zip(mats, outs):
        assert torch.equal(o, affine_gemv(m, xd, out_dtype=torch.float32))
    outs16 = affine_gemv_multi(mats, xd, out_dtype=torch.bfloat16)
    for m, o in zip(mats, outs16):
        assert torch.equal(o, affine_gemv(m, xd, out_dtype=torch.bfloat16))
    w, sc, bi = host[0]
    for r in (0, M - 1):
        ref = oracle.affine_gemv(bf16_to_f32(xb[r]), w, sc, bi, shapes[0][0], I, bits, 64)
        assert normwise_rel(outs[0].cpu().numpy()[r], ref) <= 2e-5


def test_gemv_multi_rejects_mixed_geometry(gpu):
    import torch
    from logan_amd.device import LoganHipError, affine_gemv_multi

    rng = np.random.default_rng(3)
    a = dev_matrix(torch, *make_affine(rng, 64, 512, 4, 64), 64, 512, 4, 64)
    b = dev_matrix(torch, *make_affine(rng, 64, 1024, 4, 64), 64, 1024, 4, 64)
    c = dev_matrix(torch, *make_affine(rng, 64, 512, 8, 64), 64, 512, 8, 64)
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device="cuda")
    for bad in ([a, c], [a] * 9):
        with pytest.raises(LoganHipError):
            affine_gemv_multi(bad, x)
    with pytest.raises(Exception):
        affine_gemv_multi([a, b], x)


def test_host_route_island_survives_calls_between_begin_and_finish(gpu):
    """The reference's caller runs the shared expert (and may run other
    GEMVs) between begin and finish (backend_metal.mm:3745-3747). Here:
    begin A, shared expert, a dense matmul, begin B on other experts, finish
    B, then finish A: every output against the oracle."""
    from logan_amd import backend

    rng = np.random.default_rng(123)
    D, M, bits, gs = 2048, 512, 4, 64

    def expert_descs(k):
        descs, mats = [], []
        for _ in range(k):
            g = make_affine(rng, M, D, bits, gs)
            u = make_affine(rng, M, D, bits, gs)
            d = make_affine(rng, D, M, bits, gs)
            mats.append((g, u, d))
            for (w, sc, bi), (o, i) in ((g, (M, D)), (u, (M, D)), (d, (D, M))):
                descs.append(backend.MlxAffineMatmulDesc(backend.Tensor(), np.zeros(0, np.float32),
                                                         w, aux_bytes(sc, bi), bits, gs, False, i, o))
        return descs, mats

    xa = bf16_to_f32(make_x(rng, D))
    xb = bf16_to_f32(make_x(rng, D))
    da, ma = expert_descs(4)
    db, mb = expert_descs(2)
    ds, ms = expert_descs(1)
    pa = backend.moe_route_begin(da, xa, D, M)
    assert pa is not None
    sh = np.zeros(D, np.float32)
    assert backend.shared_expert(ds, xa, sh, D, M) is True
    (wg, scg, big) = make_affine(rng, 1000, D, bits, gs)
    y = np.zeros(1000, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul_mlx_affine(t, y, xa, wg, aux_bytes(scg, big), bits, gs, False, D, 1000)
    pb = backend.moe_route_begin(db, xb, D, M)
    assert pb is not None
    outb = np.zeros(2 * D, np.float32)
    assert backend.moe_route_finish(pb, outb) == 1
    outa = np.zeros(4 * D, np.float32)
    assert backend.moe_route_finish(pa, outa) == 1
    for e, (g, u, d) in enumerate(ma):
        assert normwise_rel(outa[e * D:(e + 1) * D], _expert_ref(xa, g, u, d, D, M, bits, gs)) < 1e-4
    for e, (g, u, d) in enumerate(mb):
        assert normwise_rel(outb[e * D:(e + 1) * D], _expert_ref(xb, g, u, d, D, M, bits, gs)) < 1e-4
    g, u, d = ms[0]
    assert normwise_rel(sh, _expert_ref(xa, g, u, d, D, M, bits, gs)) < 1e-4
    assert normwise_rel(y, oracle.affine_gemv(xa, wg, scg, big, 1000, D, bits, gs)) < 1e-4
    t.free()
    for dsc in da + db + ds:
        dsc.tensor.free()


def test_host_multi_fast_and_exact_paths(gpu):
    """coli_metal_matmul_multi with f32 host activations: products the bf16
    kernels take run there on (hi, lo) activation pairs, the rest (group
    size 16 here) on the exact per-element kernel; shared and private
    activations with several rows each. Every row against the oracle's f32
    GEMV within 2e-5 normwise, the reference CUDA twin's bar
    (logan-qwen4/src/lib.rs:17176): both paths sum in another order than the
    oracle's sequential loop."""
    import ctypes as C
    from logan_amd import _lib as L
    from logan_amd.backend import Tensor

    rng = np.random.default_rng(314)
    S = 4
    specs = [  # (O, I, bits, gs, private rows or 0 for the shared x)
        (300, 2048, 4, 64, 0), (96, 2048, 5, 16, 0), (130, 1024, 8, 64, 3), (77, 512, 6, 32, 2),
        (4096, 2048, 4, 64, 0)]
    xs = bf16_to_f32(make_x(rng, S, 2048)).reshape(S, 2048) + np.float32(1e-3) * \
        rng.standard_normal((S, 2048)).astype(np.float32)  # not bf16-exact: lo halves matter
    raw = (L.MatmulDesc * len(specs))()
    keep, mats, ys, privs = [], [], [], []
    for k, (O, I, bits, gs, rows) in enumerate(specs):
        w, sc, bi = make_affine(rng, O, I, bits, gs)
        aux = aux_bytes(sc, bi)
        n = rows if rows else S
        y = np.zeros((n, O), np.float32)
        xp = None
        if rows:
            xp = (rng.standard_normal((rows, I)) * 0.7).astype(np.float32)
            privs.append(xp)
        raw[k].tensor = None
        raw[k].y = y.ctypes.data
        raw[k].weights = w.ctypes.data
        raw[k].scales = aux.ctypes.data
        raw[k].fmt = {4: 16, 5: 17, 6: 18, 8: 19}[bits]
        raw[k].I, raw[k].O, raw[k].gs = I, O, gs
        raw[k].x = xp.ctypes.data if rows else None
        raw[k].S = rows
        keep += [w, aux]
        mats.append((w, sc, bi, O, I, bits, gs))
        ys.append((y, xp))
    xs_c = np.ascontiguousarray(xs[:, :2048])
    assert L.lib().logan_hip_matmul_multi(xs_c.ctypes.data, S, raw, len(specs)) == 1
    for k, ((w, sc, bi, O, I, bits, gs), (y, xp)) in enumerate(zip(mats, ys)):
        xin = xp if xp is not None else xs_c[:, :I]
        for r in range(xin.shape[0]):
            ref = oracle.affine_gemv(np.ascontiguousarray(xin[r]), w, sc, bi, O, I, bits, gs)
            err = normwise_rel(y[r], ref)
            assert err <= 2e-5, f"desc {k} row {r}: {err:.2e}"
    for k in range(len(specs)):
        Tensor(raw[k].tensor or 0).free()


SWIGLU_SHAPES = [
    # (O, I, bits, gs): config 2's gate/up (8-bit 4096 -> 14336, cut to a
    # slice of rows), the expert shape of config 3, short and odd rows, 5/6-bit
    (3000, 4096, 8, 64), (512, 2048, 4, 64), (200, 512, 5, 64), (96, 1024, 6, 128),
    (77, 256, 4, 32), (1000, 16384, 4, 64),
]


@pytest.mark.parametrize("O,I,bits,gs", SWIGLU_SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 33])
def test_gemv_swiglu_matches_oracle(gpu, O, I, bits, gs, M):
    """h = silu(gate . x) * (up . x) in one product (logan_hip_affine_gemv_swiglu)
    against the oracle's f32 GEMVs and silu_mul, f32 h within 5e-5 normwise,
    bf16 h equal to RNE of the f32 h; M = 33 crosses the 32-token pass."""
    import torch
    from logan_amd.device import affine_gemv_swiglu

    print(f"swiglu O={O} I={I} bits={bits} gs={gs} M={M}", flush=True)
    rng = np.random.default_rng(O * 7 + I + bits + M)
    g = make_affine(rng, O, I, bits, gs)
    u = make_affine(rng, O, I, bits, gs)
    xb = make_x(rng, M, I).reshape(M, I)
    gm, um = dev_matrix(torch, *g, O, I, bits, gs), dev_matrix(torch, *u, O, I, bits, gs)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    h = affine_gemv_swiglu(gm, um, x, out_dtype=torch.float32)
    hb = affine_gemv_swiglu(gm, um, x, out_dtype=torch.bfloat16)
    assert torch.equal(hb, h.to(torch.bfloat16))
    h = h.cpu().numpy()
    for m in range(M):
        xf = bf16_to_f32(xb[m])
        yg = oracle.affine_gemv(xf, *g, O, I, bits, gs)
        yu = oracle.affine_gemv(xf, *u, O, I, bits, gs)
        ref = oracle.silu_mul(yg, yu)
        assert normwise_rel(h[m], ref) <= 5e-5, m


FULLK_SHAPES = [
    # (O, I, bits, gs, fp16): gate/up pairs with >= 12288 rows take the full-K
    # kernel at 3..16 tokens: config 2's 4096 -> 14336 at 8-bit, 4/5/6-bit,
    # a row count that is not a multiple of the 64-row block, groups of 128
    # (scale/bias per step, not per 512-code run), fp16 sidecars
    (14336, 4096, 8, 64, False), (12288, 1024, 4, 64, False), (12300, 512, 5, 64, False),
    (12352, 1024, 6, 128, False), (12288, 1536, 4, 64, True),
]


@pytest.mark.parametrize("O,I,bits,gs,fp16", FULLK_SHAPES)
@pytest.mark.parametrize("M", [3, 4, 8, 16, 17, 33])
def test_gemv_swiglu_full_k_matches_oracle(gpu, O, I, bits, gs, fp16, M):
    """The gate/up + SwiGLU product over the full K (no partial sums, h
    formed in the kernel) against the oracle's f32 GEMVs and silu_mul: f32 h
    within 5e-5 normwise, bf16 h equal to RNE of the f32 h. M = 17 and 33
    take the K-split pair (and the dot2 kernel for the 33rd token)."""
    import torch
    from logan_amd.device import affine_gemv_swiglu

    print(f"swiglu full-K O={O} I={I} bits={bits} gs={gs} fp16={fp16} M={M}", flush=True)
    rng = np.random.default_rng(O + I * 3 + bits + M + int(fp16))
    g = make_affine(rng, O, I, bits, gs, fp16)
    u = make_affine(rng, O, I, bits, gs, fp16)
    xb = make_x(rng, M, I).reshape(M, I)
    gm = dev_matrix(torch, *g, O, I, bits, gs, fp16)
    um = dev_matrix(torch, *u, O, I, bits, gs, fp16)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    h = affine_gemv_swiglu(gm, um, x, out_dtype=torch.float32)
    hb = affine_gemv_swiglu(gm, um, x, out_dtype=torch.bfloat16)
    assert torch.equal(hb, h.to(torch.bfloat16))
    h = h.cpu().numpy()
    for m in range(M):
        xf = bf16_to_f32(xb[m])
        ref = oracle.silu_mul(oracle.affine_gemv(xf, *g, O, I, bits, gs, fp16=fp16),
                              oracle.affine_gemv(xf, *u, O, I, bits, gs, fp16=fp16))
        assert normwise_rel(h[m], ref) <= 5e-5, m
