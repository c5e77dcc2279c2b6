"""GPU parity of the MFMA prefill product (logan_hip_affine_qmm) against the
oracle's restatement of the reference QMM (backend_metal.mm:1480-1560:
bf16-rounded dequantised weights, f32 accumulation).

Bars: f32 output within max|y-ŷ|/max|ŷ| <= 1e-5 of the oracle (the weights
are identical bf16 values; only the f32 summation order differs); bf16 output
equal to RNE of the f32 output; rows and columns past a tile edge untouched.
"""
import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_to_f32, make_affine, make_x

from _util import normwise_rel

pytestmark = pytest.mark.gpu


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16=False):
    from logan_amd.device import AffineMatrix

    return AffineMatrix(to_dev(w, torch), to_dev(sc.view(np.int16), torch),
                        to_dev(bi.view(np.int16), torch), O, I, bits, gs, fp16)


CASES = [
    # (M, O, I, bits, gs, fp16): tile edges in M and O, every width, group sizes
    (1, 64, 64, 4, 64, False),
    (7, 100, 128, 4, 32, False),
    (64, 64, 256, 5, 64, False),
    (130, 200, 256, 6, 128, True),
    (96, 72, 192, 8, 64, False),
    (64, 512, 2048, 4, 64, False),   # config-5 attention projection shape, one tile of M
    (33, 192, 1024, 5, 32, True),
    (65, 130, 512, 8, 128, False),
    (200, 96, 320, 5, 64, False),    # large-tile kernel: M > 64, partial tiles in M and N
    (300, 257, 128, 4, 32, True),
]


@pytest.mark.parametrize("M,O,I,bits,gs,fp16", CASES,
                         ids=lambda v: str(v))
def test_qmm_matches_oracle(gpu, M, O, I, bits, gs, fp16):
    import torch
    from logan_amd.device import affine_qmm

    rng = np.random.default_rng(M * 1000 + O + bits)
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16)
    xb = make_x(rng, M, I).reshape(M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y = affine_qmm(m, x, out_dtype=torch.float32).cpu().numpy()
    ref = oracle.affine_qmm_bf16(bf16_to_f32(xb).reshape(M, I), w, sc, bi, O, I, bits, gs, fp16)
    assert normwise_rel(y, ref) <= 1e-5
    yb = affine_qmm(m, x, out_dtype=torch.bfloat16)
    assert torch.equal(yb, torch.from_numpy(y).cuda().to(torch.bfloat16))


def test_qmm_prefill_chunk(gpu):
    """M = 512 (the config-5 prefill chunk) through one 2048 x 2048 4-bit
    projection, against the oracle on a sample of output columns."""
    import torch
    from logan_amd.device import affine_qmm

    rng = np.random.default_rng(55)
    M, O, I, bits, gs = 512, 2048, 2048, 4, 64
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    xb = make_x(rng, M, I).reshape(M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y = affine_qmm(m, x, out_dtype=torch.float32).cpu().numpy()
    cols = np.arange(0, O, 61)
    ws = w.reshape(O, -1)[cols]
    ng = I // gs
    scs = sc.reshape(O, ng)[cols].reshape(-1)
    bis = bi.reshape(O, ng)[cols].reshape(-1)
    ref = oracle.affine_qmm_bf16(bf16_to_f32(xb).reshape(M, I), ws, scs, bis, len(cols), I, bits, gs)
    assert normwise_rel(y[:, cols], ref) <= 1e-5


@pytest.mark.parametrize("bits,gs,fp16", [(4, 64, False), (5, 64, True), (8, 128, False)])
def test_qmm_large_tiles_ragged(gpu, bits, gs, fp16):
    """A grid of >= 192 tiles of 128 x 128 (the large-tile kernel) with
    partial tiles in both M and N, against the oracle on a sample of output
    columns (every column of the last, partial tile included)."""
    import torch
    from logan_amd.device import affine_qmm

    rng = np.random.default_rng(bits * 3 + gs)
    M, O, I = 500, 6337, 256
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16)
    xb = make_x(rng, M, I).reshape(M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y = affine_qmm(m, x, out_dtype=torch.float32).cpu().numpy()
    cols = np.concatenate([np.arange(0, O, 53), np.arange(O - 65, O)])
    ng = I // gs
    ws = w.reshape(O, -1)[cols]
    scs = sc.reshape(O, ng)[cols].reshape(-1)
    bis = bi.reshape(O, ng)[cols].reshape(-1)
    ref = oracle.affine_qmm_bf16(bf16_to_f32(xb).reshape(M, I), ws, scs, bis, len(cols), I, bits, gs,
                                 fp16)
    assert normwise_rel(y[:, cols], ref) <= 1e-5
    yb = affine_qmm(m, x, out_dtype=torch.bfloat16)
    assert torch.equal(yb, torch.from_numpy(y).cuda().to(torch.bfloat16))


def test_qmm_leaves_outside_untouched(gpu):
    """A y with a wider stride: columns beyond O keep their contents."""
    import torch
    from logan_amd.device import AffineMatrix
    from logan_amd import _lib as L
    import ctypes as C

    rng = np.random.default_rng(9)
    M, O, I, bits, gs = 40, 70, 128, 4, 64
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    x = to_dev(make_x(rng, M, I).reshape(M, I).view(np.int16), torch).view(torch.bfloat16)
    y = torch.full((M, 80), 7.0, dtype=torch.float32, device="cuda")
    a = m.c()
    rc = L.lib().logan_hip_affine_qmm(C.byref(a), x.data_ptr(), M, I, y.data_ptr(), 80,
                                      L.LOGAN_HIP_F32, None)
    torch.cuda.synchronize()
    assert rc == 1
    assert torch.all(y[:, O:] == 7.0)


@pytest.mark.parametrize("O,I", [(64, 2048), (512, 2048), (2048, 4096), (8192, 2048)],
                         ids=["ba", "k_v", "o_out", "q"])
def test_qmm_config5_prefill_projections(gpu, O, I):
    """The config-5 projections at the prefill chunk M = 512: grids with few
    tiles split K (ordered f32 partials and a reduction launch), large grids
    take the double-buffered 128 x 128 kernel. Sampled output columns against
    the oracle; two calls give identical bits."""
    import torch
    from logan_amd.device import affine_qmm

    print(f"qmm config5 O={O} I={I}", flush=True)
    rng = np.random.default_rng(O + I)
    M, bits, gs = 512, 4, 64
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    xb = make_x(rng, M, I).reshape(M, I)
    m = dev_matrix(torch, w, sc, bi, O, I, bits, gs)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    y = affine_qmm(m, x, out_dtype=torch.float32)
    y2 = affine_qmm(m, x, out_dtype=torch.float32)
    assert torch.equal(y, y2)
    yb = affine_qmm(m, x, out_dtype=torch.bfloat16)
    assert torch.equal(yb, y.to(torch.bfloat16))
    y = y.cpu().numpy()
    cols = np.unique(np.concatenate([np.arange(0, O, max(1, O // 24)), [O - 1]]))
    ng = I // gs
    ws = w.reshape(O, -1)[cols]
    scs = sc.reshape(O, ng)[cols].reshape(-1)
    bis = bi.reshape(O, ng)[cols].reshape(-1)
    ref = oracle.affine_qmm_bf16(bf16_to_f32(xb).reshape(M, I), ws, scs, bis, len(cols), I, bits, gs)
    assert normwise_rel(y[:, cols], ref) <= 1e-5


MULTI_CASES = [
    # (M, [O_i], I, bits, gs, fp16)
    (512, [8192, 512, 512], 2048, 4, 64, False),   # config-5 q / k / v in one grid
    (512, [12288, 64], 2048, 4, 64, False),        # config-5 qkvz / ba
    (300, [100, 257, 64], 192, 5, 64, True),       # ragged tiles, 5-bit runs at bit 16
    (256, [130, 72], 512, 6, 128, False),
    (384, [200, 96, 40, 33], 256, 8, 32, False),
    (270, [96, 64], 192, 4, 96, False),            # group size 96: one launch per matrix
    (64, [128, 96], 256, 4, 64, False),            # M < 256: one launch per matrix
]


KSLAB_CASES = [
    # grids short of 192 tiles of 256 x 128 with K a multiple of 1024: 64 x 64
    # tiles, K split across the 8 waves of a block (2, 4 or 6 steps per wave)
    (300, [2048], 1024, 5, 32, True),
    (270, [200, 130], 2048, 6, 128, False),        # ragged N and M
    (511, [1000], 3072, 8, 64, False),
    (256, [64, 96, 40], 1024, 4, 64, True),
    (257, [520, 33], 2048, 4, 32, False),          # one row in the last M tile
]

MULTI_CASES += KSLAB_CASES


@pytest.mark.parametrize("M,Os,I,bits,gs,fp16", MULTI_CASES, ids=lambda v: str(v))
def test_qmm_multi_matches_oracle(gpu, M, Os, I, bits, gs, fp16):
    """Matrices that share x in one product launch (logan_hip_affine_qmm_multi):
    every output against the oracle (sampled columns of the wide ones, every
    column of each last tile), the bf16 outputs equal to RNE of the f32 ones,
    and repeated calls identical."""
    import torch
    from logan_amd.device import affine_qmm_multi

    print(f"qmm multi M={M} Os={Os} I={I} bits={bits} gs={gs}", flush=True)
    rng = np.random.default_rng(M + sum(Os) + bits)
    mats, devs = [], []
    for O in Os:
        w, sc, bi = make_affine(rng, O, I, bits, gs, fp16)
        mats.append((w, sc, bi))
        devs.append(dev_matrix(torch, w, sc, bi, O, I, bits, gs, fp16))
    xb = make_x(rng, M, I).reshape(M, I)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    ys = affine_qmm_multi(devs, x, out_dtype=torch.float32)
    ys2 = affine_qmm_multi(devs, x, out_dtype=torch.float32)
    ybs = affine_qmm_multi(devs, x, out_dtype=torch.bfloat16)
    xf = bf16_to_f32(xb).reshape(M, I)
    ng = I // gs
    for (w, sc, bi), O, y, y2, yb in zip(mats, Os, ys, ys2, ybs):
        assert torch.equal(y, y2)
        assert torch.equal(yb, y.to(torch.bfloat16))
        cols = np.unique(np.concatenate([np.arange(0, O, max(1, O // 40)),
                                         np.arange(max(0, O - 130), O)]))
        ws = w.reshape(O, -1)[cols]
        scs = sc.reshape(O, ng)[cols].reshape(-1)
        bis = bi.reshape(O, ng)[cols].reshape(-1)
        ref = oracle.affine_qmm_bf16(xf, ws, scs, bis, len(cols), I, bits, gs, fp16)
        assert normwise_rel(y.cpu().numpy()[:, cols], ref) <= 1e-5, O


def test_split_qmm_on_three_overlapping_streams(gpu):
    """Split-K products pass their partial sums through 2 library-owned
    slots. Three streams, each issuing four split products back to back
    with no synchronisation between the streams, so more calls are in flight
    than there are slots: every output equals the single-stream result
    bitwise (the kernels are deterministic), and one per stream matches the
    oracle."""
    import torch
    from logan_amd.device import affine_gemv, affine_qmm

    M, O, I, bits, gs = 64, 512, 4096, 4, 64  # 8 tiles: the grid splits K
    mats, xs, hosts = [], [], []
    for s in range(3):
        rng = np.random.default_rng(900 + s)
        w, sc, bi = make_affine(rng, O, I, bits, gs)
        xb = make_x(rng, M, I).reshape(M, I)
        mats.append(dev_matrix(torch, w, sc, bi, O, I, bits, gs))
        xs.append(to_dev(xb.view(np.int16), torch).view(torch.bfloat16))
        hosts.append((w, sc, bi, xb))
    serial = [affine_qmm(mats[s], xs[s], out_dtype=torch.float32) for s in range(3)]
    serial_g = [affine_gemv(mats[s], xs[s][:8], out_dtype=torch.float32) for s in range(3)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(3)]
    outs = [[torch.full((M, O), float("nan"), device="cuda") for _ in range(4)] for _ in range(3)]
    outs_g = [[torch.full((8, O), float("nan"), device="cuda") for _ in range(4)] for _ in range(3)]
    torch.cuda.synchronize()
    for r in range(4):
        for s in range(3):
            with torch.cuda.stream(streams[s]):
                affine_qmm(mats[s], xs[s], out=outs[s][r], stream=streams[s])
                affine_gemv(mats[s], xs[s][:8], out=outs_g[s][r], stream=streams[s])
    torch.cuda.synchronize()
    for s in range(3):
        for r in range(4):
            assert torch.equal(outs[s][r], serial[s]), (s, r)
            assert torch.equal(outs_g[s][r], serial_g[s]), (s, r)
        w, sc, bi, xb = hosts[s]
        cols = np.arange(0, O, 37)
        ng = I // gs
        ref = oracle.affine_qmm_bf16(bf16_to_f32(xb).reshape(M, I), w.reshape(O, -1)[cols],
                                     sc.reshape(O, ng)[cols].reshape(-1),
                                     bi.reshape(O, ng)[cols].reshape(-1), len(cols), I, bits, gs)
        assert normwise_rel(serial[s].cpu().numpy()[:, cols], ref) <= 1e-5
