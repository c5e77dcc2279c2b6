"""GPU parity of the dense Llama decode layer (coli_metal_llama_layer and the
device-native logan_hip_llama_layer) and the raw-bf16 GEMV against the CPU
oracle (logan-llama/src/model.rs:786-905).

Bars: the layer's x, K and V rows within max|y-ŷ| <= 1e-4 * max|ŷ| of the
oracle at every position (f32 residual stream; the GPU forms the products
from bf16 hi/lo activation halves and sums in another order); fmt 15 and
fmt 5 with the loader's bf16 weights bitwise equal on the GPU; the bf16
GEMV within 2e-5 normwise of the oracle.
"""
import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32

from _util import normwise_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


def make_layer(rng, D, inter, H, KH, hd, fmts):
    """7 matrices (fmt per matrix) plus the float32 dequantised copies."""
    shapes = [(H * hd, D), (KH * hd, D), (KH * hd, D), (D, H * hd), (inter, D), (inter, D),
              (D, inter)]
    mats = []
    for (O, I), fmt in zip(shapes, fmts):
        scale = 1.0 / np.sqrt(I)
        if fmt == 5:
            w = bf16_bits((rng.standard_normal((O, I)) * scale).astype(np.float32))
            mats.append((5, w, None, None))
        else:
            codes = rng.integers(0, 256, (O, I)).astype(np.uint8)
            s = (np.abs(rng.standard_normal((O, I // 64))) * scale / 40 + scale / 200).astype(np.float32)
            sc = bf16_bits(s)
            bi = bf16_bits((-128 * bf16_to_f32(sc)).astype(np.float32))
            mats.append((15, codes, sc, bi))
    return mats


def loader_bf16(codes, sc, bi):
    """logan-llama's load-time dequantisation (weights.rs:441-516)."""
    deq = codes.astype(np.float32) * np.repeat(bf16_to_f32(sc), 64, axis=1) + \
        np.repeat(bf16_to_f32(bi), 64, axis=1)
    return bf16_bits(deq.astype(np.float32))


def host_descs(backend, mats):
    out = []
    for fmt, w, sc, bi in mats:
        O, I = w.shape
        aux = np.zeros(1, np.uint8) if fmt == 5 else np.concatenate([sc.reshape(-1), bi.reshape(-1)]).view(np.uint8)
        out.append(backend.MetalMatmulDesc(backend.Tensor(), np.zeros(0, np.float32), w, aux, fmt, I, O))
    return out


def rel(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.mark.parametrize("fmts", [(5,) * 7, (15,) * 7, (15, 5, 15, 5, 15, 5, 15)],
                         ids=["bf16", "affine8", "mixed"])
def test_host_llama_layer_matches_oracle(gpu, fmts):
    """coli_metal_llama_layer over 12 positions of one layer; x, K and V of
    every position against the oracle carrying its own cache."""
    from logan_amd import backend

    rng = np.random.default_rng(sum(fmts))
    D, inter, H, KH, hd, theta, eps = 256, 512, 8, 2, 32, 500000.0, 1e-5
    mats = make_layer(rng, D, inter, H, KH, hd, fmts)
    descs = host_descs(backend, mats)
    in_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    post_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    T = 12
    kc = np.zeros((T, KH * hd), np.float32)
    vc = np.zeros((T, KH * hd), np.float32)
    model = 42
    try:
        for pos in range(T):
            x = rng.standard_normal(D).astype(np.float32)
            want = oracle.llama_layer(x, kc, vc, pos, mats, in_norm, post_norm, D, inter, H, KH, hd,
                                      theta, eps)
            k_out = np.zeros(KH * hd, np.float32)
            v_out = np.zeros(KH * hd, np.float32)
            rc = backend.llama_layer(model, 3, descs, x, k_out, v_out, in_norm, post_norm, D, inter,
                                     H, KH, hd, pos, theta, eps)
            assert rc == 1, pos
            assert rel(x, want) < TOL, (pos, rel(x, want))
            assert rel(k_out, kc[pos]) < TOL and rel(v_out, vc[pos]) < TOL, pos
    finally:
        backend.llama_drop_model(model)
        for d in descs:
            d.tensor.free()


def test_host_llama_layer_reference_tiny_model(gpu):
    """The reference's tiny test model (logan-llama/tests/oracle_parity.rs
    :1-100), tokens 1, 2, 3 decoded one by one: each step's x against the
    oracle."""
    from logan_amd import backend

    D, inter, H, KH, hd = 4, 8, 2, 1, 2
    shapes = [(H * hd, D), (KH * hd, D), (KH * hd, D), (D, H * hd), (inter, D), (inter, D), (D, inter)]
    consts = [0.1, 0.1, 0.1, 0.1, 0.02, 0.03, 0.02]
    # D = 4 is not a multiple of 16: the dense kernel declines that width
    descs = host_descs(backend, [(5, np.full(s, bf16_bits(np.array([c], np.float32))[0], np.uint16), None, None)
                                 for s, c in zip(shapes, consts)])
    ones = np.ones(D, np.float32)
    x = np.arange(4, 8, dtype=np.float32) / 20
    rc = backend.llama_layer(7, 0, descs, x, np.zeros(2, np.float32), np.zeros(2, np.float32), ones,
                             ones, D, inter, H, KH, hd, 0, 10000.0, 1e-5)
    assert rc == 0 and np.all(x == np.arange(4, 8, dtype=np.float32) / 20)
    backend.llama_drop_model(7)


def test_host_llama_layer_positions_and_drop(gpu):
    """Calls must come in position order (the reference declines otherwise,
    backend_metal.mm:2643); drop_model resets the context; a changed norm
    pointer or geometry for the same (model, layer) declines."""
    from logan_amd import backend

    rng = np.random.default_rng(2)
    D, inter, H, KH, hd = 128, 256, 4, 4, 32
    mats = make_layer(rng, D, inter, H, KH, hd, (5,) * 7)
    descs = host_descs(backend, mats)
    n1 = np.ones(D, np.float32)
    n2 = np.ones(D, np.float32)
    k = np.zeros(KH * hd, np.float32)
    v = np.zeros(KH * hd, np.float32)

    def call(pos, x=None, norm=n1, model=9, heads=H):
        x = rng.standard_normal(D).astype(np.float32) if x is None else x
        return backend.llama_layer(model, 0, descs, x, k, v, norm, norm, D, inter, heads, KH, hd,
                                   pos, 10000.0, 1e-5)

    try:
        assert call(1) == 0  # must start at 0
        assert call(0) == 1
        assert call(0) == 0  # position 0 again: out of order
        assert call(1) == 1
        assert call(2, norm=n2) == 0  # another norm array for the same layer
        backend.llama_drop_model(9)
        assert call(0) == 1
        # a first call on layer 0 of another model, then its own order
        assert call(0, model=10) == 1 and call(1, model=10) == 1
        # bad descriptors: wrong orientation declines before anything runs
        bad = list(descs)
        bad[4], bad[6] = descs[6], descs[4]
        x = np.ones(D, np.float32)
        assert backend.llama_layer(11, 0, bad, x, k, v, n1, n1, D, inter, H, KH, hd, 0, 1e4, 1e-5) == 0
        assert np.all(x == 1)
    finally:
        backend.llama_drop_model(9)
        backend.llama_drop_model(10)
        for d in descs:
            d.tensor.free()


def _dev_layer(torch, mats, in_norm, post_norm, cap, D, inter, H, KH, hd, theta, eps):
    from logan_amd.device import DenseMatrix, LlamaLayer

    dm = []
    for fmt, w, sc, bi in mats:
        O, I = w.shape
        wt = torch.from_numpy(np.ascontiguousarray(w).view(np.int16 if fmt == 5 else np.uint8)).cuda()
        if fmt == 5:
            dm.append(DenseMatrix(wt, O, I, 5))
        else:
            dm.append(DenseMatrix(wt, O, I, 15, torch.from_numpy(sc.view(np.int16)).cuda(),
                                  torch.from_numpy(bi.view(np.int16)).cuda()))
    kvd = KH * hd
    return LlamaLayer(dm, torch.from_numpy(in_norm).cuda(), torch.from_numpy(post_norm).cuda(),
                      torch.zeros((cap, kvd), dtype=torch.float32, device="cuda"),
                      torch.zeros((cap, kvd), dtype=torch.float32, device="cuda"),
                      D, inter, H, KH, hd, theta, eps)


def test_device_llama_layer_config2_shape(gpu):
    """logan_hip_llama_layer at the dense config-2 shape (D 4096, 32 heads over
    8 kv heads of 128, inter 14336, affine-8 g64) at position 5 over a cache
    of earlier rows: x, K and V against the oracle; then the same layer with
    the loader's bf16 weights (fmt 5) gives bitwise the same x."""
    import torch

    from logan_amd.device import llama_layer

    rng = np.random.default_rng(2048)
    D, inter, H, KH, hd, theta, eps = 4096, 14336, 32, 8, 128, 500000.0, 1e-5
    mats = make_layer(rng, D, inter, H, KH, hd, (15,) * 7)
    in_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    post_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    pos, cap = 5, 8
    kc = np.zeros((cap, KH * hd), np.float32)
    vc = np.zeros((cap, KH * hd), np.float32)
    kc[:pos] = rng.standard_normal((pos, KH * hd)).astype(np.float32)
    vc[:pos] = rng.standard_normal((pos, KH * hd)).astype(np.float32)
    x = rng.standard_normal(D).astype(np.float32)
    kc_o, vc_o = kc.copy(), vc.copy()
    want = oracle.llama_layer(x, kc_o, vc_o, pos, mats, in_norm, post_norm, D, inter, H, KH, hd,
                              theta, eps)
    layer = _dev_layer(torch, mats, in_norm, post_norm, cap, D, inter, H, KH, hd, theta, eps)
    layer.k_cache.copy_(torch.from_numpy(kc))
    layer.v_cache.copy_(torch.from_numpy(vc))
    xd = torch.from_numpy(x).cuda()
    llama_layer(layer, xd, pos)
    got = xd.cpu().numpy()
    assert rel(got, want) < TOL
    assert rel(layer.k_cache[pos].cpu().numpy(), kc_o[pos]) < TOL
    assert rel(layer.v_cache[pos].cpu().numpy(), vc_o[pos]) < TOL
    # earlier rows untouched
    assert torch.equal(layer.k_cache[:pos].cpu(), torch.from_numpy(kc[:pos]))
    # the same weights as the loader's bf16 matrices (fmt 5): bitwise equal
    mats5 = [(5, loader_bf16(w, sc, bi), None, None) for _, w, sc, bi in mats]
    layer5 = _dev_layer(torch, mats5, in_norm, post_norm, cap, D, inter, H, KH, hd, theta, eps)
    layer5.k_cache.copy_(torch.from_numpy(kc))
    layer5.v_cache.copy_(torch.from_numpy(vc))
    xd5 = torch.from_numpy(x).cuda()
    llama_layer(layer5, xd5, pos)
    assert torch.equal(xd5, xd)


def test_device_llama_layer_rejects(gpu):
    import torch

    from logan_amd.device import LoganHipError, llama_layer

    rng = np.random.default_rng(5)
    D, inter, H, KH, hd = 128, 256, 4, 2, 32
    mats = make_layer(rng, D, inter, H, KH, hd, (5,) * 7)
    ones = np.ones(D, np.float32)
    layer = _dev_layer(torch, mats, ones, ones, 4, D, inter, H, KH, hd, 1e4, 1e-5)
    x = torch.zeros(D, dtype=torch.float32, device="cuda")
    with pytest.raises(LoganHipError):  # position beyond the cache
        llama_layer(layer, x, 4)
    xo = torch.zeros(D + 1, dtype=torch.float32, device="cuda")[1:]
    with pytest.raises(LoganHipError):  # x not 16-byte aligned (read as float4)
        llama_layer(layer, xo, 0)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(LoganHipError):  # workspace not 16-byte aligned
        llama_layer(layer, x, 0, workspace=ws[8:])
    layer.head_dim = 512  # more than 256
    with pytest.raises(LoganHipError):
        llama_layer(layer, x, 0)


@pytest.mark.parametrize("S", [1, 3])
def test_host_matmul_bf16_fmt5(gpu, S):
    """coli_metal_matmul with raw bf16 weights (fmt 5, the llama loader's
    default) against the oracle's bf16 GEMV."""
    from logan_amd import backend

    rng = np.random.default_rng(50 + S)
    O, I = 1000, 1536
    w = bf16_bits((rng.standard_normal((O, I)) * 0.05).astype(np.float32))
    x = rng.standard_normal(S * I).astype(np.float32)
    y = np.zeros(S * O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul(t, y, x, w, np.ones(1, np.float32), 5, I, O, 0, S)
    assert t.nbytes() == O * I * 2
    for s in range(S):
        want = oracle.dense_gemv(x[s * I:(s + 1) * I], w, O, I, 5)
        assert normwise_rel(y[s * O:(s + 1) * O], want) < 2e-5
    t.free()
