"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against the reference's own known-answer
vectors (tests/golden/kat_vectors.json) and against arithmetic that shares
nothing with the oracle's code path: numpy bit unpacking, float64 matmuls of
the dequantised matrix, exhaustive fp16 decoding, torch's bf16 rounding,
numpy's stable argsort, closed forms. A planted mistake (wrong shift, dropped
bias, transposed index, reversed tie rule) fails at least one of them.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32, make_affine, make_logits, make_x

from _util import dequant_f64, pack_codes, unpack_codes

import test_mxfp4_gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "kat_vectors.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["decode"], ids=lambda c: f"{c['source'].split(':')[-1]}-b{c['bits']}")
def test_dequant_matches_reference_kat(case):
    words = np.array(case["words"], dtype=np.uint32)
    sc = bf16_bits(np.array(case["scales"], np.float32))
    bi = bf16_bits(np.array(case["biases"], np.float32))
    got = oracle.affine_dequant(words.view(np.uint8), sc, bi, case["rows"], case["cols"],
                                case["bits"], case["group_size"])
    np.testing.assert_array_equal(got.reshape(-1), np.array(case["expected"], np.float32))


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_code_extraction_bruteforce(bits):
    """Every column of random rows, including every straddling position."""
    rng = np.random.default_rng(bits)
    I = 256
    codes = rng.integers(0, 1 << bits, size=(3, I))
    packed = pack_codes(codes, bits)
    np.testing.assert_array_equal(unpack_codes(packed, I, bits), codes)
    for r in range(3):
        got = [oracle.affine_code(packed[r], c, bits) for c in range(I)]
        np.testing.assert_array_equal(got, codes[r])


def test_f16_decode_exhaustive():
    lib = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.lo_f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_bf16_rne_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.0e38, -3.0e38, 1e-40],
                 np.float32),
        # exact ties: low 16 bits == 0x8000 with even and odd kept LSB
        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000], np.uint32)).view(np.float32),
    ])
    lib = oracle.lib()
    got = np.array([lib.lo_f32_to_bf16(float(v)) for v in vals], np.uint16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(bf16_bits(vals), want)


@pytest.mark.parametrize("bits,gs,fp16", [(4, 64, False), (5, 128, False), (6, 64, False),
                                          (8, 128, False), (4, 32, True), (8, 64, True)])
def test_dequant_matches_independent_decode(bits, gs, fp16):
    rng = np.random.default_rng(10 + bits)
    O, I = 5, 256
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16=fp16)
    got = oracle.affine_dequant(w, sc, bi, O, I, bits, gs, fp16=fp16)
    want = dequant_f64(w, sc, bi, O, I, bits, gs, fp16)
    # code*scale is exact in f32 and adding the bias rounds once
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_dequant_rejects_bad_geometry():
    w = np.zeros(64, np.uint8)
    sc = np.zeros(4, np.uint16)
    with pytest.raises(ValueError):
        oracle.affine_dequant(w, sc, sc, 1, 60, 4, 32)  # 60 % 32 != 0
    with pytest.raises(ValueError):
        oracle.affine_dequant(w, sc, sc, 1, 64, 7, 32)  # unsupported width


@pytest.mark.parametrize("case", GOLDEN["gemv"], ids=lambda c: f"b{c['bits']}")
def test_gemv_reference_closed_forms(case):
    O, I, bits, gs = case["O"], case["I"], case["bits"], case["group_size"]
    w = np.full((O, I * bits // 8), case["byte"], np.uint8)
    sc = bf16_bits(np.full(O * (I // gs), case["scale"], np.float32))
    bi = bf16_bits(np.full(O * (I // gs), case["bias"], np.float32))
    x = np.full(I, case["x"], np.float32)
    y = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs, nthreads=1)
    np.testing.assert_array_equal(y, np.full(O, case["expected"], np.float32))


def test_spark_affine8_reference_closed_form():
    c = GOLDEN["spark_affine8"]
    O, I = c["O"], c["I"]
    aux = np.concatenate([bf16_bits(np.full(O, c["scale"], np.float32)),
                          bf16_bits(np.full(O, c["bias"], np.float32))])
    y = oracle.spark_affine8_gemv(np.full(I, c["x"], np.float32), np.full(O * I, c["byte"], np.uint8),
                                  aux, O, I)
    np.testing.assert_array_equal(y, np.full(O, c["expected"], np.float32))


def _spark_case(rng, O, I):
    """Integer codes, integer x and power-of-two scales/biases that differ per
    (row, group): every product and partial sum is exact in f32, so the
    expected accumulator is exact and only the final bf16 rounding is left."""
    ng = I // 64
    codes = rng.integers(0, 256, (O, I)).astype(np.uint8)
    x = rng.integers(-3, 4, I).astype(np.float32)
    sc = np.float32([0.25, 0.5, 1.0, 2.0])[rng.integers(0, 4, (O, ng))]
    bi = np.float32([-32.0, -8.0, 4.0, 24.0])[rng.integers(0, 4, (O, ng))]
    return codes, x, sc, bi


def _spark_expected(codes, x, sc, bi, bias=True, row_params=True):
    O, I = codes.shape
    acc = np.zeros(O, np.float64)
    for r in range(O):
        pr = r if row_params else 0
        for g in range(I // 64):
            s = slice(64 * g, 64 * g + 64)
            acc[r] += sc[pr, g] * float(codes[r, s].astype(np.float64) @ x[s])
            if bias:
                acc[r] += bi[pr, g] * float(x[s].sum())
    return acc


def test_spark_affine8_closed_form_bias_and_rounding():
    """logan-spark/src/lib.rs:346-367: acc = sum_g sc[r,g] * dot_g + bi[r,g] *
    xsum[g], then bf16 RNE. With exact accumulators the oracle must equal
    torch's bf16 rounding of the exact value; the case is built so that a
    dropped bias term, row-0 parameters for every row, or no rounding all
    give different outputs."""
    rng = np.random.default_rng(41)
    O, I = 16, 256
    codes, x, sc, bi = _spark_case(rng, O, I)
    aux = np.concatenate([bf16_bits(sc.ravel()), bf16_bits(bi.ravel())])
    y = oracle.spark_affine8_gemv(x, codes.ravel(), aux, O, I)
    exact = _spark_expected(codes, x, sc, bi)
    assert np.all(np.abs(exact) < 2.0 ** 24)  # exact in f32
    want = _bf16_round_torch(exact.astype(np.float32))
    np.testing.assert_array_equal(y, want)
    # the case separates the plausible mistakes
    assert np.sum(want != exact.astype(np.float32)) >= O // 2  # rounding visible
    assert np.sum(_bf16_round_torch(_spark_expected(codes, x, sc, bi, bias=False)
                                    .astype(np.float32)) != want) >= O - 1
    assert np.sum(_bf16_round_torch(_spark_expected(codes, x, sc, bi, row_params=False)
                                    .astype(np.float32)) != want) >= O - 2


def test_spark_affine8_random_against_float64():
    """Random codes, bf16 N(0,1) x and make_affine's bf16 scale/bias: the
    oracle is within 1 bf16 ulp of RNE(float64 dequant-then-dot), and equal
    to it for nearly every row (f32 accumulation only moves outputs that sit
    next to a rounding boundary)."""
    rng = np.random.default_rng(42)
    O, I = 256, 4096
    w, sc, bi = make_affine(rng, O, I, 8, 64)
    x = bf16_to_f32(make_x(rng, 1, I))[0]
    aux = np.concatenate([sc, bi])
    y = oracle.spark_affine8_gemv(x, w.ravel(), aux, O, I)
    ref64 = dequant_f64(w, sc, bi, O, I, 8, 64) @ x.astype(np.float64)
    want = _bf16_round_torch(ref64.astype(np.float32))
    ulp = np.abs(want) * 2.0 ** -7
    assert np.all(np.abs(y - want) <= ulp * 1.0001)
    assert np.mean(y == want) >= 0.95


@pytest.mark.parametrize("bits,gs", [(4, 64), (5, 128), (6, 64), (8, 128)])
def test_gemv_reference_generator_against_float64(bits, gs):
    """The generator of logan-metal/src/lib.rs:1310-1378 (codes
    (17r+7c+3)&mask, scale 0.125(r+g+1), bias -0.25+0.0625(r+g),
    x ((i%11)-5)*0.125), checked with that test's own tolerance
    max(2e-3, 2e-4|ref|) against a float64 matmul of the decoded matrix."""
    O, I = 3, 128
    mask = (1 << bits) - 1
    codes = np.array([[(r * 17 + c * 7 + 3) & mask for c in range(I)] for r in range(O)])
    w = pack_codes(codes, bits)
    g = I // gs
    sc = bf16_bits(np.array([[0.125 * (r + q + 1) for q in range(g)] for r in range(O)], np.float32))
    bi = bf16_bits(np.array([[-0.25 + 0.0625 * (r + q) for q in range(g)] for r in range(O)], np.float32))
    x = np.array([((i % 11) - 5) * 0.125 for i in range(I)], np.float32)
    y = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs, nthreads=1)
    ref = dequant_f64(w, sc, bi, O, I, bits, gs) @ x.astype(np.float64)
    tol = np.maximum(2e-3, 2e-4 * np.abs(ref))
    assert np.all(np.abs(y - ref) <= tol)


@pytest.mark.parametrize("bits,gs,fp16", [(4, 64, False), (5, 64, False), (6, 64, False),
                                          (8, 64, False), (4, 128, True)])
def test_gemv_random_against_float64(bits, gs, fp16):
    rng = np.random.default_rng(bits * 7)
    O, I = 64, 1024
    w, sc, bi = make_affine(rng, O, I, bits, gs, fp16=fp16)
    x = bf16_to_f32(make_x(rng, I))
    y1 = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs, fp16, nthreads=1)
    y8 = oracle.affine_gemv(x, w, sc, bi, O, I, bits, gs, fp16, nthreads=8)
    np.testing.assert_array_equal(y1, y8)  # row split leaves each row's order intact
    ref = dequant_f64(w, sc, bi, O, I, bits, gs, fp16) @ x.astype(np.float64)
    assert np.abs(y1 - ref).max() / np.abs(ref).max() < 1e-5


def test_softmax_matches_float64():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(512).astype(np.float32) * 3
    p = oracle.softmax_row(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5


@pytest.mark.parametrize("seed", range(6))
def test_topk_matches_stable_argsort(seed):
    rng = np.random.default_rng(seed)
    E, k = 512, 10
    logits = bf16_to_f32(make_logits(rng, 1, E, zipf_s=1.1 if seed % 2 else None)[0])
    if seed >= 4:
        # force ties straddling the k-th place
        order = np.argsort(-logits, kind="stable")
        logits[order[7:14]] = logits[order[8]]
    probs = oracle.softmax_row(logits)
    idx, val, wsum = oracle.topk(probs, k)
    want = np.argsort(-probs, kind="stable")[:k]  # descending prob, lower index first
    np.testing.assert_array_equal(idx, want)
    np.testing.assert_array_equal(val, probs[want])
    assert wsum == pytest.approx(float(probs[want].astype(np.float64).sum()), rel=1e-6)


def test_topk_tie_rule_prefers_lower_index():
    probs = np.array([0.1, 0.3, 0.3, 0.05, 0.3, 0.25], np.float32)
    idx, _, _ = oracle.topk(probs, 4)
    np.testing.assert_array_equal(idx, [1, 2, 4, 5])


def _moe_f64(x, logits, k, D, inter, bits, gs, gate, up, down, shared, se_g):
    """Float64 statement of the MoE block for the oracle check."""
    x64 = x.astype(np.float64)
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    idx = np.argsort(-p, kind="stable")[:k]
    w = p[idx] / p[idx].sum()
    out = np.zeros(D)

    def mlp(g_, u_, d_, e, hi):
        G = dequant_f64(g_[0][e], g_[1][e], g_[2][e], hi, D, bits, gs)
        U = dequant_f64(u_[0][e], u_[1][e], u_[2][e], hi, D, bits, gs)
        Dn = dequant_f64(d_[0][e], d_[1][e], d_[2][e], D, hi, bits, gs)
        gv, uv = G @ x64, U @ x64
        h = gv / (1 + np.exp(-gv)) * uv
        return Dn @ h

    for r in range(k):
        out += w[r] * mlp(gate, up, down, idx[r], inter)
    if shared is not None:
        gsig = 1 / (1 + np.exp(-(se_g.astype(np.float64) @ x64)))
        sg, su, sd = shared
        out += gsig * mlp((sg[0][None], sg[1][None], sg[2][None]),
                          (su[0][None], su[1][None], su[2][None]),
                          (sd[0][None], sd[1][None], sd[2][None]), 0, inter)
    return out, idx, w


@pytest.mark.parametrize("bits", [4, 6])
def test_moe_token_against_float64(bits):
    rng = np.random.default_rng(100 + bits)
    E, k, D, inter, gs = 16, 4, 128, 64, 64
    gate = make_affine(rng, inter, D, bits, gs, E=E)
    up = make_affine(rng, inter, D, bits, gs, E=E)
    down = make_affine(rng, D, inter, bits, gs, E=E)
    shared = (make_affine(rng, inter, D, bits, gs), make_affine(rng, inter, D, bits, gs),
              make_affine(rng, D, inter, bits, gs))
    se_g = bf16_to_f32(make_x(rng, D)) * np.float32(0.05)
    x = bf16_to_f32(make_x(rng, D))
    logits = bf16_to_f32(make_logits(rng, 1, E)[0])
    out, idx, w = oracle.moe_token(x, logits, k, D, inter, bits, gs, gate, up, down, shared, se_g)
    ref, ridx, rw = _moe_f64(x, logits, k, D, inter, bits, gs, gate, up, down, shared, se_g)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=1e-5)
    assert np.abs(out - ref).max() / np.abs(ref).max() < 1e-4


def test_moe_expert_source_closed_form():
    """logan-qwen4/src/lib.rs:17277-17348: expert 0 (zero codes) gives 0,
    expert 1 (code 1, scale 1, bias 0, x = 1, D = M = 64) gives
    64 * silu(64) * 64 per element."""
    c = GOLDEN["expert"]
    D = M = c["D"]
    words = D * 4 // 32
    def bank(rows):
        w = np.empty((2, rows, words), np.uint32)
        w[0] = c["expert0_word"]
        w[1] = c["expert1_word"]
        sc = bf16_bits(np.full((2, rows, 1), c["scale"], np.float32))
        bi = bf16_bits(np.full((2, rows, 1), c["bias"], np.float32))
        return w.view(np.uint8).reshape(2, rows, -1), sc, bi
    gate, up, down = bank(M), bank(M), bank(D)
    x = np.full(D, c["x"], np.float32)
    for expert, want in ((0, c["expected_expert0"]), (1, c["expected_expert1"])):
        logits = np.array([0.0, 0.0], np.float32)
        logits[expert] = 10.0
        out, idx, w = oracle.moe_token(x, logits, 1, D, M, 4, 64, gate, up, down)
        assert idx[0] == expert and w[0] == 1.0
        if want == 0.0:
            assert np.all(out == 0.0)
        else:
            assert np.all(np.abs(out - want) <= abs(want) * c["rel_tol"])


def _bf16_round_torch(a: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def test_qmm_closed_form():
    """Constant code 3, scale bf16(0.1), bias 0: every weight is bf16(3 * 0.1)
    (not 3 * 0.1) and y = 64 * that weight for x = 1 (exact in f32)."""
    M, O, I, bits, gs = 2, 4, 64, 8, 64
    w = np.full((O, I), 3, np.uint8)
    sc = bf16_bits(np.full(O * (I // gs), 0.1, np.float32))
    bi = bf16_bits(np.zeros(O * (I // gs), np.float32))
    y = oracle.affine_qmm_bf16(np.ones((M, I), np.float32), w, sc, bi, O, I, bits, gs)
    wq = _bf16_round_torch(np.float32(3.0) * bf16_to_f32(sc[:1]))[0]
    assert wq != np.float32(3.0) * bf16_to_f32(sc[:1])[0]  # the rounding is visible
    np.testing.assert_array_equal(y, np.full((M, O), 64 * wq, np.float32))


@pytest.mark.parametrize("bits,gs", [(4, 64), (5, 32), (6, 128), (8, 64)])
def test_qmm_against_float64_of_bf16_weights(bits, gs):
    """The prefill oracle equals a float64 product of the bf16-rounded
    (torch RNE) float64 dequantisation, to f32 accumulation error; without
    the rounding it would sit ~1e-3 away."""
    rng = np.random.default_rng(bits * 13 + gs)
    M, O, I = 5, 48, 512
    w, sc, bi = make_affine(rng, O, I, bits, gs)
    x = bf16_to_f32(make_x(rng, M, I)).reshape(M, I)
    y = oracle.affine_qmm_bf16(x, w, sc, bi, O, I, bits, gs)
    wd = dequant_f64(w, sc, bi, O, I, bits, gs)
    wq = _bf16_round_torch(wd.astype(np.float32)).astype(np.float64)
    ref = x.astype(np.float64) @ wq.T
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-5
    unrounded = x.astype(np.float64) @ wd.T
    assert np.abs(unrounded - ref).max() / np.abs(ref).max() > 1e-4


def test_silu_mul_closed_form():
    """silu(g) * u against the float64 closed form g / (1 + e^-g) * u, and
    the values the formula fixes exactly: silu(0) = 0, silu(v) -> v for large
    v, silu(v) -> -0 for very negative v, u = 0 gives 0."""
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = oracle.silu_mul(g, u)
    g64 = g.astype(np.float64)
    ref = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 4e-7 * np.abs(ref) + 1e-30)
    special = oracle.silu_mul(np.array([0.0, 100.0, -200.0, 3.0], np.float32),
                              np.array([5.0, 2.0, 1.0, 0.0], np.float32))
    assert special[0] == 0.0 and special[1] == 200.0
    assert special[2] == 0.0 and special[3] == 0.0


def test_rmsnorm_closed_form_and_float64():
    """Constant rows c with eps = 0 normalise to sign(c) * w exactly (c a power
    of two: mean(x^2) = c^2 exact); random rows match a float64 statement of
    x / sqrt(mean(x^2) + eps) * w. A missing 1/n, a dropped eps or weights
    applied per row instead of per column fail one of these."""
    w = np.arange(1, 9, dtype=np.float32) * np.float32(0.5)
    x = np.stack([np.full(8, 4.0, np.float32), np.full(8, -0.25, np.float32)])
    np.testing.assert_array_equal(oracle.rmsnorm(x, w, 0.0), np.stack([w, -w]))
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 2048)).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32)
    eps = 1e-5
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
    got = oracle.rmsnorm(x, w, eps)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    # eps matters where the rows are small
    tiny = np.full((1, 2048), 1e-3, np.float32)
    assert not np.allclose(oracle.rmsnorm(tiny, w, 1e-5), oracle.rmsnorm(tiny, w, 0.0))


def test_add_is_elementwise_sum():
    rng = np.random.default_rng(8)
    y = rng.standard_normal(1000).astype(np.float32)
    a = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.add(y, a), y + a)


def test_mxfp4_canonical_nibble_order_kat():
    """logan-qwen4/src/lib.rs:17676-17694: bytes 0x10 0x32 .. 0xfe at scale
    byte 127 hold 0, 0.5, .., 6, -0, .., -6, element 2j in the low nibble."""
    c = GOLDEN["mxfp4_order"]
    got = []
    for b in c["bytes"]:
        got += [oracle.mxfp4_value(b & 0xF, c["scale_byte"]), oracle.mxfp4_value(b >> 4, c["scale_byte"])]
    np.testing.assert_array_equal(np.float32(got).view(np.uint32),
                                  np.float32(c["expected"]).view(np.uint32))
    # the same bytes through the GEMV with one-hot x pick each element
    O, I = 1, 16
    w = np.array(c["bytes"], np.uint8)
    for col in range(I):
        x = np.zeros(I, np.float32)
        x[col] = 1.0
        y = oracle.mxfp4_gemv(x, w, np.array([c["scale_byte"]], np.uint8), O, I)
        assert y[0] == c["expected"][col]


@pytest.mark.parametrize("case", GOLDEN["mxfp4_gemv"], ids=lambda c: hex(c["byte"]))
def test_mxfp4_reference_projection_closed_forms(case):
    """logan-qwen4/src/lib.rs:17604-17651: constant code bytes, scale 1."""
    O, I = case["O"], case["I"]
    y = oracle.mxfp4_gemv(np.float32(case["x"]), np.full(O * I // 2, case["byte"], np.uint8),
                          np.full(O * I // 32, case["scale_byte"], np.uint8), O, I)
    np.testing.assert_array_equal(y, np.full(O, case["expected"], np.float32))


def test_mxfp4_decode_exhaustive_against_float64():
    """Every code under a range of scale bytes: sign * E2M1 magnitude *
    2^(byte - 127), with the E2M1 magnitudes rebuilt from the format (exponent
    bits e, mantissa bit m: m/2 for e = 0, else 2^(e-1) (1 + m/2))."""
    for code in range(16):
        e, m, neg = (code >> 1) & 3, code & 1, code & 8
        mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        for sb in (1, 64, 100, 126, 127, 128, 130, 200, 254):
            want = (-mag if neg else mag) * 2.0 ** (sb - 127)
            got = oracle.mxfp4_value(code, sb)
            with np.errstate(over="ignore"):  # 6 * 2^127 is inf in f32, as in the reference
                assert got == np.float32(want) and np.signbit(got) == bool(neg), (code, sb)


@pytest.mark.parametrize("stacks", [1, 2, 3])
def test_mxfp4_gemv_random_against_float64(stacks):
    """Random bytes and scale bytes near 127, stacked planes (fmt 7/9/10):
    the oracle against a float64 decode-then-dot of the summed planes; a
    swapped nibble order or a dropped residual plane fails it."""
    rng = np.random.default_rng(70 + stacks)
    O, I = 40, 512
    w = rng.integers(0, 256, (stacks, O, I // 2)).astype(np.uint8)
    sc = rng.integers(120, 131, (stacks, O, I // 32)).astype(np.uint8)
    x = rng.standard_normal(I).astype(np.float32)

    def dec(wp, sp, swap=False):
        lo, hi = (wp >> 4, wp & 0xF) if swap else (wp & 0xF, wp >> 4)
        codes = np.stack([lo, hi], axis=-1).reshape(O, I)
        tab = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
        return tab[codes] * np.repeat(2.0 ** (sp.astype(np.float64) - 127), 32, axis=1)

    ref = sum(dec(w[s], sc[s]) for s in range(stacks)) @ x.astype(np.float64)
    y = oracle.mxfp4_gemv(x, w, sc, O, I, stacks)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    swapped = sum(dec(w[s], sc[s], True) for s in range(stacks)) @ x.astype(np.float64)
    assert np.abs(swapped - ref).max() > 1e-2 * np.abs(ref).max()
    if stacks > 1:
        first = dec(w[0], sc[0]) @ x.astype(np.float64)
        assert np.abs(first - ref).max() > 1e-2 * np.abs(ref).max()


# ---- dense Llama decode layer ---------------------------------------------


def _bf16v(v):
    return bf16_to_f32(bf16_bits(np.array([v], np.float32)))[0]


def _tiny_llama():
    """The reference's own test model (logan-llama/tests/oracle_parity.rs
    :1-100): D 4, inter 8, 2 heads over 1 kv head of dim 2, constant bf16
    weights, unit norms, embedding row t = (4t .. 4t+3) / 20."""
    D, inter, H, KH, hd = 4, 8, 2, 1, 2
    shapes = [(H * hd, D), (KH * hd, D), (KH * hd, D), (D, H * hd), (inter, D), (inter, D),
              (D, inter)]
    consts = [0.1, 0.1, 0.1, 0.1, 0.02, 0.03, 0.02]
    mats = [(5, np.full(s, bf16_bits(np.float32(c)), np.uint16), None, None)
            for s, c in zip(shapes, consts)]
    return D, inter, H, KH, hd, mats, consts


def test_llama_tiny_model_closed_form():
    """Two decode steps of the reference's tiny model against a float64
    closed form: every projection of a constant-weight matrix is c * sum(in),
    RoPE at pos 0 is the identity and at pos 1 rotates (a, a) by 1 rad, one
    kv head serves both heads, and att is the softmax mix of the cached v."""
    D, inter, H, KH, hd, mats, consts = _tiny_llama()
    eps, theta = 1e-5, 10000.0
    cq, ck, cv, co, cg, cu, cd = (float(_bf16v(c)) for c in consts)
    kc = np.zeros((2, KH * hd), np.float32)
    vc = np.zeros((2, KH * hd), np.float32)
    ones = np.ones(D, np.float32)

    def rms(v):
        return v / np.sqrt(np.mean(v * v) + eps)

    def mlp(x1):
        pn = rms(x1)
        g, u = cg * pn.sum(), cu * pn.sum()
        h = g / (1 + np.exp(-g)) * u
        return x1 + cd * inter * h

    ks, vs, qs = [], [], []
    for pos, tok in enumerate((1, 2)):
        x = np.arange(4 * tok, 4 * tok + 4, dtype=np.float64) / 20
        xf = np.float32(x)
        got = oracle.llama_layer(xf, kc, vc, pos, mats, ones, ones, D, inter, H, KH, hd, theta, eps)
        s = rms(x).sum()
        q0, k0, v0 = cq * s, ck * s, cv * s
        c, si = np.cos(pos), np.sin(pos)  # angle pos / theta^0 for the single pair
        q = np.array([q0 * c - q0 * si, q0 * si + q0 * c])
        k = np.array([k0 * c - k0 * si, k0 * si + k0 * c])
        ks.append(k)
        vs.append(np.array([v0, v0]))
        sc = np.array([q @ kk / np.sqrt(hd) for kk in ks])
        p = np.exp(sc - sc.max())
        p /= p.sum()
        att = sum(pp * vv for pp, vv in zip(p, vs))  # [hd], same for both heads
        x1 = x + co * 2 * att.sum()  # o row: c * sum over both heads' att
        want = mlp(x1)
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(kc[pos], k, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(vc[pos], [v0, v0], rtol=2e-6, atol=1e-7)


def _np_llama_f64(x, kc, vc, pos, Ws, in_norm, post_norm, H, KH, hd, theta, eps):
    """float64 decode layer in the Hugging Face formulation (rotate_half RoPE
    with inv_freq = theta^(-2i/hd); repeat_kv grouping), written from the
    model's definition: the independent check of the oracle."""
    x = x.astype(np.float64)

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v) + eps) * w

    def rope(v, n):
        v = v.reshape(n, hd)
        inv = theta ** (-np.arange(0, hd, 2) / hd)
        ang = np.concatenate([pos * inv, pos * inv])
        rot = np.concatenate([-v[:, hd // 2:], v[:, :hd // 2]], axis=1)
        return (v * np.cos(ang) + rot * np.sin(ang)).reshape(-1)

    Wq, Wk, Wv, Wo, Wg, Wu, Wd = Ws
    xn = rms(x, in_norm)
    q, k, v = rope(Wq @ xn, H), rope(Wk @ xn, KH), Wv @ xn
    K = np.vstack([kc[:pos].astype(np.float64), k[None]]).reshape(pos + 1, KH, hd)
    V = np.vstack([vc[:pos].astype(np.float64), v[None]]).reshape(pos + 1, KH, hd)
    K, V = np.repeat(K, H // KH, axis=1), np.repeat(V, H // KH, axis=1)
    qh = q.reshape(H, hd)
    s = np.einsum("hd,thd->ht", qh, K) / np.sqrt(hd)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    att = np.einsum("ht,thd->hd", p, V).reshape(-1)
    x1 = x + Wo @ att
    pn = rms(x1, post_norm)
    g, u = Wg @ pn, Wu @ pn
    return x1 + Wd @ (g / (1 + np.exp(-g)) * u), k, v


@pytest.mark.parametrize("fmt", [5, 15])
def test_llama_layer_against_float64_model(fmt):
    """Six positions of a random layer (4 heads over 2 kv heads of dim 16)
    against the float64 Hugging Face formulation. A half-split RoPE taken as
    interleaved pairs, h % KH grouping, a missing 1/sqrt(hd) or a dropped
    residual each fail it."""
    rng = np.random.default_rng(11 + fmt)
    D, inter, H, KH, hd, theta, eps = 64, 128, 4, 2, 16, 10000.0, 1e-6
    shapes = [(H * hd, D), (KH * hd, D), (KH * hd, D), (D, H * hd), (inter, D), (inter, D),
              (D, inter)]
    mats, Ws = [], []
    for O, I in shapes:
        if fmt == 5:
            w = bf16_bits((rng.standard_normal((O, I)) * 0.15).astype(np.float32))
            mats.append((5, w, None, None))
            Ws.append(bf16_to_f32(w).astype(np.float64))
        else:
            codes = rng.integers(0, 256, (O, I)).astype(np.uint8)
            sc = bf16_bits((np.abs(rng.standard_normal((O, I // 64))) * 0.002 + 1e-4).astype(np.float32))
            bi = bf16_bits((-128 * bf16_to_f32(sc)).astype(np.float32))
            mats.append((15, codes, sc, bi))
            deq = codes * np.repeat(bf16_to_f32(sc), 64, axis=1) + np.repeat(bf16_to_f32(bi), 64, axis=1)
            Ws.append(bf16_to_f32(bf16_bits(deq.astype(np.float32))).astype(np.float64))
    in_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    post_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    T = 6
    kc = np.zeros((T, KH * hd), np.float32)
    vc = np.zeros((T, KH * hd), np.float32)
    for pos in range(T):
        x = rng.standard_normal(D).astype(np.float32)
        got = oracle.llama_layer(x, kc, vc, pos, mats, in_norm, post_norm, D, inter, H, KH, hd,
                                 theta, eps)
        want, k, v = _np_llama_f64(x, kc, vc, pos, Ws, in_norm.astype(np.float64),
                                   post_norm.astype(np.float64), H, KH, hd, theta, eps)
        assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max(), pos
        np.testing.assert_allclose(kc[pos], k, rtol=0, atol=2e-5 * np.abs(k).max())
        np.testing.assert_allclose(vc[pos], v, rtol=0, atol=2e-5 * np.abs(v).max())


def test_dense_gemv_fmt15_equals_fmt5_of_loader_weights():
    """fmt 15 forms each weight as RNE_bf16(code * scale + bias), which is the
    bf16 matrix logan-llama's loader stores (weights.rs:441-516): the two
    products agree bit for bit."""
    rng = np.random.default_rng(3)
    O, I = 24, 256
    codes = rng.integers(0, 256, (O, I)).astype(np.uint8)
    sc = bf16_bits((np.abs(rng.standard_normal((O, I // 64))) * 0.01).astype(np.float32))
    bi = bf16_bits((rng.standard_normal((O, I // 64)) * 0.5).astype(np.float32))
    deq = codes.astype(np.float32) * np.repeat(bf16_to_f32(sc), 64, axis=1) + \
        np.repeat(bf16_to_f32(bi), 64, axis=1)
    w5 = bf16_bits(deq.astype(np.float32))
    x = rng.standard_normal(I).astype(np.float32)
    a = oracle.dense_gemv(x, codes, O, I, 15, sc, bi)
    b = oracle.dense_gemv(x, w5, O, I, 5)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = bf16_to_f32(w5).astype(np.float64) @ x.astype(np.float64)
    assert np.abs(a - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("planes", [1, 3])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_full_range_case_is_what_it_claims(planes, xdt):
    """CPU: the planted rows give the oracle outputs the GPU test relies on."""
    w, sc, x, want = test_mxfp4_gpu.full_range_case(planes, xdt)
    O = want.shape[0]
    if planes == 1:
        assert want[0] == np.inf and np.isnan(want[1:5]).all() and want[5] == np.inf
    assert (want[6:8] == 0).all()
    assert np.isnan(want[:O // 2]).any() and np.isinf(want[:O // 2]).any()
    assert np.isfinite(want[O // 2:]).all()
    assert (sc[:, O // 2:] <= 40).any() and (sc == 0).any() and (sc == 255).any()
