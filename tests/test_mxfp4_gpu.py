"""GPU parity of the MXFP4 paths (logan-metal fmt 7, residual planes fmt 9 /
10) against the CPU oracle.

Bars: decoded weights bit-exact (sign of zero included); f32 outputs within
max|y-ŷ| <= 2e-5 * max_r sum_j |w_rj x_j| of the oracle's f32 GEMV (the
reference orders its per-element f32 sums differently from both, and the f32
activation enters as bf16 hi + lo, |x - hi - lo| <= 2^-18 |x|); bf16 outputs
equal to RNE of the same kernel's f32 output. The host drop-in paths
(coli_metal_matmul, route island, shared_mxfp4) are held to the reference
tests' 2e-5 / 1e-4 normwise figures (logan-qwen4/src/lib.rs:17164-17173).
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32

from _util import normwise_rel

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "kat_vectors.json").read_text())
MX4 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])


def make_mx(rng, O, I, planes=1, lo=118, hi=136):
    w = rng.integers(0, 256, (planes, O, I // 2)).astype(np.uint8)
    sc = rng.integers(lo, hi, (planes, O, I // 32)).astype(np.uint8)
    return w, sc


def abs_dot(w, sc, x, O, I):
    """max_r sum_j |w_rj x_j| over the summed planes (float64), the scale of
    the accumulation error bound."""
    tot = np.zeros((O, I))
    for p in range(w.shape[0]):
        codes = np.stack([w[p] & 0xF, w[p] >> 4], axis=-1).reshape(O, I)
        tot += np.abs(MX4[codes] * np.repeat(2.0 ** (sc[p].astype(np.float64) - 127), 32, axis=1))
    return float((tot @ np.abs(x.astype(np.float64))).max())


def dev_mx(torch, w, sc, O, I):
    from logan_amd.device import Mxfp4Matrix

    return Mxfp4Matrix(torch.from_numpy(np.ascontiguousarray(w)).cuda(),
                       torch.from_numpy(np.ascontiguousarray(sc)).cuda(), O, I, w.shape[0])


def same_bits_or_nan(got, want):
    """f32 arrays equal bit for bit, except that a NaN only has to be a NaN
    (its payload and sign are the platform's: 0 * inf is 0x7FC00000 on the
    GPU, 0xFFC00000 on x86)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_mxfp4_dequant_bit_exact(gpu):
    """The decode instruction against the oracle, every code under every scale
    byte 0..255 (the golden canonical-order bytes first), sign of zero
    included; byte 0 is a zero scale, byte 255 an infinite one (zero codes
    then decode to NaN, as the reference's product gives)."""
    import torch

    from logan_amd.device import mxfp4_dequant

    rng = np.random.default_rng(7)
    O, I = 96, 512
    w, sc = make_mx(rng, O, I, 1, 0, 256)
    sc[0, 1:, :2] = [0, 255]  # every row holds both extremes
    c = GOLDEN["mxfp4_order"]
    w[0, 0, :8] = c["bytes"]
    sc[0, 0, 0] = c["scale_byte"]
    got = mxfp4_dequant(dev_mx(torch, w, sc, O, I)).cpu().numpy()
    np.testing.assert_array_equal(got[0, :16].view(np.uint32),
                                  np.float32(c["expected"]).view(np.uint32))
    lib = oracle.lib()
    want = np.empty((O, I), np.float32)
    for r in range(O):
        for j in range(I):
            b = int(w[0, r, j // 2])
            want[r, j] = lib.lo_mxfp4_value(b & 0xF if j % 2 == 0 else b >> 4, int(sc[0, r, j // 32]))
    assert np.isnan(want).any() and np.isinf(want).any() and (want[:, :32] == 0).any()
    same_bits_or_nan(got, want)
    # a row window
    part = mxfp4_dequant(dev_mx(torch, w, sc, O, I), 37, 5).cpu().numpy()
    same_bits_or_nan(part, want[37:42])


@pytest.mark.parametrize("planes", [1, 2, 3])
@pytest.mark.parametrize("O,I", [(1, 32), (37, 256), (512, 2048), (2048, 512), (96, 4096)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_mxfp4_gemv_matches_oracle(gpu, planes, O, I, xdt):
    import torch

    from logan_amd.device import mxfp4_gemv

    rng = np.random.default_rng(planes * 1000 + O + I)
    w, sc = make_mx(rng, O, I, planes)
    if xdt == "f32":
        x = rng.standard_normal(I).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
    else:
        xb = bf16_bits(rng.standard_normal(I).astype(np.float32))
        x = bf16_to_f32(xb)
        xd = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    want = oracle.mxfp4_gemv(x, w, sc, O, I, planes)
    m = dev_mx(torch, w, sc, O, I)
    (y,) = mxfp4_gemv([m], [xd])
    y = y.cpu().numpy()
    bound = 2e-5 * abs_dot(w, sc, x, O, I)
    assert np.abs(y - want).max() <= bound
    # bf16 output: the same f32 sum rounded once (RNE)
    (yb,) = mxfp4_gemv([m], [xd], out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(yb.cpu().view(torch.int16).numpy().view(np.uint16), bf16_bits(y))


def row_abs_dot(w, sc, x, O, I):
    """sum_j |w_rj x_j| per row over the summed planes (float64)."""
    tot = np.zeros(O)
    ax = np.abs(x.astype(np.float64))
    for p in range(w.shape[0]):
        codes = np.stack([w[p] & 0xF, w[p] >> 4], axis=-1).reshape(O, I)
        wa = np.abs(MX4[codes] * np.repeat(2.0 ** (sc[p].astype(np.float64) - 127), 32, axis=1))
        tot += wa @ ax
    return tot


def full_range_case(planes, xdt):
    """Scale bytes over all of 0..255 (see test_mxfp4_gemv_full_scale_range):
    (w, sc, x, want) with the oracle's output."""
    rng = np.random.default_rng(2550 + planes + (xdt == "bf16"))
    O, I = 320, 1024
    w, sc = make_mx(rng, O, I, planes, 0, 256)
    sc[:, O // 2:] = rng.integers(0, 201, sc[:, O // 2:].shape)
    sc[0, :8] = rng.integers(110, 140, (8, I // 32))  # planted rows: moderate elsewhere
    x = rng.standard_normal(I).astype(np.float32)
    x[:32] = np.abs(x[:32]) + np.float32(0.5)  # group 0: positive, >= 0.5
    x[96:128] = np.abs(x[96:128]) + np.float32(0.5)
    x[100] = 0.0                               # group 3: positive but one zero
    if xdt == "bf16":
        x = bf16_to_f32(bf16_bits(x))
    pos = rng.integers(1, 8, (8, 16)).astype(np.uint8)  # codes 1..7: positive, nonzero
    w[0, :8, :16] = pos | (pos << 4)
    sc[0, 0, 0] = 255                       # +inf
    sc[0, 1, 0] = 255
    w[0, 1, 5] &= 0xF0                      # one zero code -> NaN
    sc[0, 2, 3] = 255                       # group 3 holds x[100] = 0 -> NaN
    w[0, 2, 48:64] = pos[2] | (pos[2] << 4)
    sc[0, 3, 0] = 255
    w[0, 3, 7] |= 0x08                      # one negative code -> NaN
    sc[0, 4, 0] = 254
    w[0, 4, 3] = 0x7F                       # 6 and -6 at 2^127: both overflow -> NaN
    sc[0, 5, 0] = 254                       # 6 * x * 2^127 with x >= 0.5 -> +inf
    w[0, 5, :16] = 0x77
    for r in (6, 7):                        # byte-0 groups only: exact zeros
        sc[:, r] = 0
    want = oracle.mxfp4_gemv(x, w, sc, O, I, planes)
    return w, sc, x, want


@pytest.mark.parametrize("planes", [1, 3])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_mxfp4_gemv_full_scale_range(gpu, planes, xdt):
    """Scale bytes over all of 0..255 against the reference's per-element
    product (acc += x * MX4[code] * scale, logan-qwen4/src/lib.rs:2948-2961):
    where the oracle's row is NaN or +-inf the kernel's is the same, finite
    rows within 2e-5 of the row's sum_j |w_rj x_j| (plus 1e-40 for terms in
    the subnormal range, which the reference rounds one by one). Rows 0-5
    plant byte-255 groups: all codes nonzero and positive with x > 0 (+inf),
    one zero code, a zero x, codes of both signs (NaN each); byte-254 groups
    whose terms overflow with both signs (NaN) and with one sign (+inf); rows
    6-7 hold only byte-0 groups (zero); the other rows of the first half draw
    bytes from 0..255, the second half from 0..200 (finite rows with tiny
    and zero scales)."""
    import torch

    from logan_amd.device import mxfp4_gemv

    w, sc, x, want = full_range_case(planes, xdt)
    O, I = want.shape[0], x.shape[0]
    m = dev_mx(torch, w, sc, O, I)
    if xdt == "f32":
        xd = torch.from_numpy(x).cuda()
    else:
        xd = torch.from_numpy(bf16_bits(x).view(np.int16)).cuda().view(torch.bfloat16)
    (y,) = mxfp4_gemv([m], [xd])
    y = y.cpu().numpy()
    np.testing.assert_array_equal(np.isnan(y), np.isnan(want))
    inf = np.isinf(want)
    np.testing.assert_array_equal(y[inf], want[inf])
    fin = np.isfinite(want)
    bound = 2e-5 * row_abs_dot(w, sc, x, O, I)[fin] + 1e-40
    assert (np.abs(y[fin].astype(np.float64) - want[fin]) <= bound).all()
    (yb,) = mxfp4_gemv([m], [xd], out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(yb.cpu().view(torch.int16).numpy().view(np.uint16), bf16_bits(y))


def test_mxfp4_gemv_batch_of_sixteen(gpu):
    """16 matrices of mixed shapes and plane counts, each with its own x, in
    one launch: each within the bound of its oracle product, and a repeat of
    the launch bitwise equal."""
    import torch

    from logan_amd.device import mxfp4_gemv

    rng = np.random.default_rng(99)
    shapes = [(64, 32), (300, 1024), (17, 2048), (1024, 64), (5, 96), (128, 4096), (33, 512),
              (256, 256), (1, 1024), (77, 160), (2048, 128), (9, 2048), (640, 640), (48, 32),
              (100, 3072), (512, 512)]
    ms, xs, wants, ws = [], [], [], []
    for k, (O, I) in enumerate(shapes):
        planes = 1 + k % 3
        w, sc = make_mx(rng, O, I, planes)
        x = rng.standard_normal(I).astype(np.float32)
        ms.append(dev_mx(torch, w, sc, O, I))
        xs.append(torch.from_numpy(x).cuda())
        wants.append(oracle.mxfp4_gemv(x, w, sc, O, I, planes))
        ws.append((w, sc, x, O, I))
    ys = mxfp4_gemv(ms, xs)
    for k in range(16):
        w, sc, x, O, I = ws[k]
        y = ys[k].cpu().numpy()
        assert np.abs(y - wants[k]).max() <= 2e-5 * abs_dot(w, sc, x, O, I), k
    again = mxfp4_gemv(ms, xs)
    for a, b in zip(ys, again):
        assert torch.equal(a, b)


def test_mxfp4_gemv_rejects_bad_geometry(gpu):
    import torch

    from logan_amd.device import LoganHipError, Mxfp4Matrix, mxfp4_gemv

    w = torch.zeros(64 * 24, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(64 * 2, dtype=torch.uint8, device="cuda")
    x = torch.zeros(48, dtype=torch.float32, device="cuda")
    with pytest.raises(LoganHipError):  # I not a multiple of 32
        mxfp4_gemv([Mxfp4Matrix(w, sc, 64, 48)], [x])
    with pytest.raises(LoganHipError):  # four planes
        mxfp4_gemv([Mxfp4Matrix(w, sc, 16, 32, 4)], [x[:32]])


def _mx_desc(backend, rng, o, i, fmt, x=None):
    planes = backend.MXFP4_PLANES[fmt]
    w, sc = make_mx(rng, o, i, planes)
    y = np.zeros(o, np.float32)
    return backend.MetalWeightDesc(backend.Tensor(), w, sc, fmt, 0, i, o, y, x), w, sc


@pytest.mark.parametrize("fmt", [7, 9, 10])
@pytest.mark.parametrize("S", [1, 3])
def test_host_matmul_mxfp4(gpu, fmt, S):
    """coli_metal_matmul with fmt 7 / 9 / 10 through the host-pointer layer."""
    from logan_amd import backend

    rng = np.random.default_rng(fmt * 10 + S)
    O, I = 384, 1024
    planes = backend.MXFP4_PLANES[fmt]
    w, sc = make_mx(rng, O, I, planes)
    x = rng.standard_normal(S * I).astype(np.float32)
    y = np.zeros(S * O, np.float32)
    t = backend.Tensor()
    assert backend.hip_matmul(t, y, x, w, sc, fmt, I, O, 0, S)
    assert t.nbytes() == planes * O * (I // 2 + I // 32)
    for s in range(S):
        want = oracle.mxfp4_gemv(x[s * I:(s + 1) * I], w, sc, O, I, planes)
        assert normwise_rel(y[s * O:(s + 1) * O], want) < 2e-5
    # the handle is reused; a different plane count on it declines
    y2 = np.zeros_like(y)
    assert backend.hip_matmul(t, y2, x, w, sc, fmt, I, O, 0, S)
    np.testing.assert_array_equal(y, y2)
    other = {7: 9, 9: 10, 10: 7}[fmt]
    assert not backend.hip_matmul(t, y2, x, w, sc, other, I, O, 0, S)
    t.free()


def test_host_matmul_mxfp4_declines_ragged_width(gpu):
    """I not a multiple of 32: the reference serves it, this backend declines
    (the caller's CPU path runs)."""
    from logan_amd import backend

    O, I = 8, 40
    t = backend.Tensor()
    assert not backend.hip_matmul(t, np.zeros(O, np.float32), np.ones(I, np.float32),
                                  np.zeros(O * I // 2, np.uint8), np.zeros(O * 2, np.uint8), 7, I, O)
    assert t.handle == 0


def test_host_multi_mixes_mxfp4_and_affine(gpu):
    """One matmul_multi submission with MXFP4, MXFP4x3 and affine descriptors
    (shared x and a private x)."""
    from logan_amd import backend
    from logan_amd.synth import aux_bytes, make_affine

    rng = np.random.default_rng(5)
    I = 512
    x = rng.standard_normal(I).astype(np.float32)
    xp = rng.standard_normal(I).astype(np.float32)
    d7, w7, s7 = _mx_desc(backend, rng, 200, I, 7)
    d10, w10, s10 = _mx_desc(backend, rng, 64, I, 10, x=xp)
    aw, asc, abi = make_affine(rng, 128, I, 4, 64)
    da = backend.MetalWeightDesc(backend.Tensor(), aw, aux_bytes(asc, abi), 16, 64, I, 128,
                                 np.zeros(128, np.float32))
    assert backend.hip_matmul_mlx_affine_multi(x, [d7, d10, da])
    assert normwise_rel(d7.y, oracle.mxfp4_gemv(x, w7, s7, 200, I, 1)) < 2e-5
    assert normwise_rel(d10.y, oracle.mxfp4_gemv(xp, w10, s10, 64, I, 3)) < 2e-5
    assert normwise_rel(da.y, oracle.affine_gemv(x, aw, asc, abi, 128, I, 4, 64)) < 2e-5
    for d in (d7, d10, da):
        d.tensor.free()


def _mx_expert_ref(x, g, u, d, D, M):
    gv = oracle.mxfp4_gemv(x, *g, M, D, g[0].shape[0])
    uv = oracle.mxfp4_gemv(x, *u, M, D, u[0].shape[0])
    h = np.array([oracle.lib().lo_silu(float(a)) for a in gv], np.float32) * uv
    return oracle.mxfp4_gemv(h, *d, D, M, d[0].shape[0])


@pytest.mark.parametrize("K", [1, 8])
def test_host_route_island_mxfp4(gpu, K):
    """moe_route_begin/finish with fmt 7 experts (the reference's island takes
    fmt 7 and 21..24, backend_metal.mm:3749-3766): K expert outputs against
    the oracle's per-expert SwiGLU MLP."""
    from logan_amd import backend

    rng = np.random.default_rng(40 + K)
    D, M = 2048, 768
    x = bf16_to_f32(bf16_bits(rng.standard_normal(D).astype(np.float32)))
    descs, mats = [], []
    for _ in range(K):
        trio = []
        for o, i in ((M, D), (M, D), (D, M)):
            dsc, w, sc = _mx_desc(backend, rng, o, i, 7)
            descs.append(dsc)
            trio.append((w, sc))
        mats.append(trio)
    pending = backend.moe_route_begin(descs, x, D, M)
    assert pending is not None
    out = np.zeros(K * D, np.float32)
    assert backend.moe_route_finish(pending, out) == 1
    for e, (g, u, d) in enumerate(mats):
        assert normwise_rel(out[e * D:(e + 1) * D], _mx_expert_ref(x, g, u, d, D, M)) < 1e-4
    for dsc in descs:
        dsc.tensor.free()


def test_shared_mxfp4(gpu):
    """coli_metal_shared_mxfp4 with MXFP4 gate/up/down, and with an fp16
    affine down (the reference accepts fmt 7 and 21..24 per descriptor)."""
    from logan_amd import backend
    from logan_amd.synth import aux_bytes, make_affine

    rng = np.random.default_rng(123)
    D, M = 1024, 512
    x = rng.standard_normal(D).astype(np.float32)
    trio = [_mx_desc(backend, rng, o, i, 7) for o, i in ((M, D), (M, D), (D, M))]
    out = np.zeros(D, np.float32)
    assert backend.shared_mxfp4([t[0] for t in trio], x, out, D, M) is True
    want = _mx_expert_ref(x, *[(t[1], t[2]) for t in trio], D, M)
    assert normwise_rel(out, want) < 1e-4
    # fp16-sidecar affine down projection
    aw, asc, abi = make_affine(rng, D, M, 8, 64, fp16=True)
    down = backend.MetalWeightDesc(backend.Tensor(), aw, aux_bytes(asc, abi), 24, 64, M, D)
    out2 = np.zeros(D, np.float32)
    assert backend.shared_mxfp4([trio[0][0], trio[1][0], down], x, out2, D, M) is True
    gv = oracle.mxfp4_gemv(x, trio[0][1], trio[0][2], M, D)
    uv = oracle.mxfp4_gemv(x, trio[1][1], trio[1][2], M, D)
    h = np.array([oracle.lib().lo_silu(float(a)) for a in gv], np.float32) * uv
    want2 = oracle.affine_gemv(h, aw, asc, abi, D, M, 8, 64, fp16=True)
    assert normwise_rel(out2, want2) < 1e-4
    # fmt 9 is not a shared_mxfp4 format: declined before any submission
    bad = _mx_desc(backend, rng, D, M, 9)[0]
    assert backend.shared_mxfp4([trio[0][0], trio[1][0], bad], x, out2, D, M) is None
    for t in trio:
        t[0].tensor.free()
    down.tensor.free()
