"""Routing where different logits share a softmax probability.

The reference selects on probabilities p_i = fl(exp(fl(l_i - m)) / s)
(logan-qwen4/src/lib.rs:4558-4574) with lower-index ties (:8031-8040). p is
only non-decreasing in the logit, so distinct logits can tie in p:

* "subtract": tiny logits next to a large maximum, fl(l - m) rounds to the
  same exp argument (bf16 and f32 logits);
* "underflow": exp(l - m) underflows to 0 for every logit below the maximum
  (bf16 and f32);
* "neginf": -inf logits (exp 0) inside the top-k (bf16 and f32);
* "nearmax": f32 logits a few ulps below a maximum < 0.5 whose exps round to
  1.0;
* "divtie": f32 logits one ulp apart whose exps are one ulp apart and whose
  quotients by the sum round to the same probability;
* "ulp": f32 logits one ulp apart whose probabilities stay distinct (the
  recomputed selection must agree with the logit order there);
* "nan": one NaN logit makes every probability NaN; the reference's
  comparisons are then all false and it keeps experts 0..k-1;
* "prefix": f32 logits 2^-16 apart next to 2.0 (distinct probabilities,
  logit order) that share the upper bits the 32-bit selection keys keep, so
  that selection must hand over to the 64-bit keys;
* "negnan": the same with NaN bit patterns that have the sign bit set
  (0xFFC0 and others, bf16-exact): an ordered-bits key would sort such a NaN
  below every number, so the selection must treat any NaN as NaN whatever
  its sign (x86 arithmetic produces the negative default NaN).

Every case checks its own premise on the CPU: that the logit order and the
oracle's probability order really differ (where that is the point), and that
the oracle's expf agrees with a correctly rounded exp on every argument, so
the comparison does not depend on which libm computed the exps. The CPU
tests here pin the generator; the GPU tests compare route_topk and the MoE
block (every path) with the oracle, indices bit for bit.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32, make_x

from _util import normwise_rel

E, K = 512, 10
BF16_KINDS = ["subtract", "underflow", "neginf", "nan", "negnan"]
NAN_KINDS = {"nan", "negnan"}
# NaN bit patterns (f32, each bf16-exact), one per seed in turn
NEG_NANS = [0xFFC00000, 0xFF810000, 0xFFFF0000, 0x7F810000]
F32_KINDS = BF16_KINDS + ["nearmax", "divtie", "ulp", "prefix"]
ORDER_DIFFERS = {"subtract", "underflow", "neginf", "nearmax", "divtie", "nan", "negnan"}


def tie_logits(kind: str, seed: int) -> np.ndarray:
    """f32 logits [E] for one case; bf16 kinds hold bf16-exact values."""
    rng = np.random.default_rng(seed)
    lf = np.empty(E, np.float32)
    if kind == "subtract":
        lf[:] = -3.0 - 0.5 * rng.integers(0, 8, E)
        pos = np.sort(rng.choice(E, 13, replace=False))
        lf[pos[0]] = 4.0
        # 2^-27 (1 + j/16): bf16-exact, increasing with the expert index
        lf[pos[1:]] = np.float32(2.0 ** -27) * (1 + np.arange(12, dtype=np.float32) / 16)
    elif kind == "underflow":
        lf[:] = -10.0 - 0.5 * rng.integers(0, 60, E)
        lf[rng.integers(0, E)] = 100.0
    elif kind == "neginf":
        lf[:] = -np.inf
        # finite logits whose exps underflow too, between the -inf ones
        lf[1::2] = -120.0 - 2.0 * rng.integers(0, 8, E // 2)
        pos = rng.choice(E, 6, replace=False)
        lf[pos] = np.float32([3.0, 2.5, 2.0, 1.5, 1.0, 0.5])
    elif kind in ("nearmax", "divtie", "ulp", "prefix"):
        m, step = {"nearmax": (0.25, 2.0 ** -26), "divtie": (0.75, 2.0 ** -24),
                   "ulp": (2.0, 2.0 ** -22), "prefix": (2.0, 2.0 ** -16)}[kind]
        m, step = np.float32(m), np.float32(step)
        lf[:] = (m - np.float32([3.0, 4.5, 6.0, 7.5]))[rng.integers(0, 4, E)]
        pos = np.sort(rng.choice(E, 12, replace=False))
        lf[pos] = m - step * np.arange(12, dtype=np.float32)[::-1]
    elif kind == "nan":
        lf[:] = bf16_to_f32(bf16_bits(rng.standard_normal(E).astype(np.float32)))
        lf[rng.integers(0, E)] = np.nan
    elif kind == "negnan":
        lf[:] = bf16_to_f32(bf16_bits(rng.standard_normal(E).astype(np.float32)))
        pat = NEG_NANS[seed % len(NEG_NANS)]
        lf[rng.integers(K, E)] = np.uint32(pat).view(np.float32)
    else:
        raise ValueError(kind)
    return lf


def oracle_route(lf: np.ndarray, k: int):
    probs = oracle.softmax_row(lf)
    idx, val, wsum = oracle.topk(probs, k)
    return idx, (val / np.float32(wsum)).astype(np.float32)


def _libm_expf():
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    return libm.expf


@pytest.mark.parametrize("kind", F32_KINDS)
def test_tie_cases_are_what_they_claim(kind):
    """CPU: the case's premise holds for the oracle."""
    lf = tie_logits(kind, 1)
    ridx, rw = oracle_route(lf, K)
    finite = lf[np.isfinite(lf)]
    if kind not in NAN_KINDS:
        m = np.float32(finite.max())
        d = (lf - m).astype(np.float32)
        expf = _libm_expf()
        libm = np.array([expf(float(v)) for v in d], np.float32)
        with np.errstate(invalid="ignore", over="ignore"):
            cr = np.exp(d.astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(libm, cr)
    logit_order = np.argsort(-np.nan_to_num(lf, nan=np.inf), kind="stable")[:K]
    if kind in ORDER_DIFFERS:
        assert not np.array_equal(ridx, logit_order), "case does not separate the two orders"
    else:
        np.testing.assert_array_equal(ridx, logit_order)
    if kind in NAN_KINDS:
        np.testing.assert_array_equal(ridx, np.arange(K))
        assert np.isnan(rw).all()
    if kind == "negnan":
        # the planted NaN is the sign-bit kind for most seeds, below the top k,
        # and a key of its ordered bits would rank it last: the old shortcut's
        # answer (the finite logits' top k) differs from the reference's
        for seed in range(len(NEG_NANS)):
            lfs = tie_logits(kind, seed)
            pos = np.flatnonzero(np.isnan(lfs))
            assert len(pos) == 1 and pos[0] >= K
            bits = int(lfs[pos[0]:pos[0] + 1].view(np.uint32)[0])
            assert bits == NEG_NANS[seed]
            assert bf16_bits(lfs[pos])[0] == bits >> 16
        lfin = np.where(np.isnan(lf), -np.inf, lf)
        assert not np.array_equal(np.argsort(-lfin, kind="stable")[:K], ridx)


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def dev_logits(torch, lf, dtype):
    if dtype == "bf16":
        return to_dev(bf16_bits(lf).view(np.int16), torch).view(torch.bfloat16)
    return to_dev(lf, torch)


def check_route(idx, w, lf, k, kind):
    ridx, rw = oracle_route(lf, k)
    np.testing.assert_array_equal(idx, ridx)
    if kind in NAN_KINDS:
        assert np.isnan(w).all()
    elif kind == "prefix":
        # no probability tie: the fast weights exp(l_r - l_0) / sum, which
        # equal the reference's val_r / wsum up to rounding
        np.testing.assert_allclose(w, rw, rtol=2e-6, atol=0)
    else:
        # the recomputed path is the reference's arithmetic: bit-exact weights
        np.testing.assert_array_equal(w, rw)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,kind", [("bf16", k) for k in BF16_KINDS] +
                         [("f32", k) for k in F32_KINDS])
def test_route_topk_probability_ties(gpu, dtype, kind):
    import torch
    from logan_amd.device import route_topk

    B = 6
    lf = np.stack([tie_logits(kind, s) for s in range(B)])
    if dtype == "bf16":
        assert np.array_equal(bf16_to_f32(bf16_bits(lf)), lf, equal_nan=True)
    idx, w = route_topk(dev_logits(torch, lf, dtype), K)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    for b in range(B):
        print(f"route ties {dtype} {kind} token {b}", flush=True)
        check_route(idx[b], w[b], lf[b], K, kind)


MOE_TIE_CASES = [(1, "bf16", "subtract"), (1, "bf16", "underflow"), (1, "bf16", "neginf"),
                 (1, "f32", "divtie"), (1, "f32", "nearmax"), (16, "bf16", "subtract"),
                 (16, "f32", "divtie"), (64, "bf16", "underflow"), (64, "f32", "divtie"),
                 (1, "bf16", "negnan"), (1, "f32", "negnan"), (1, "bf16", "nan"),
                 (16, "bf16", "negnan"), (64, "bf16", "negnan"), (64, "f32", "negnan"),
                 (1, "f32", "prefix"), (16, "f32", "prefix"), (64, "f32", "prefix"),
                 (1, "f32", "nan")]


# B > 1 takes the multi-launch path either way: only B = 1 runs both ways
@pytest.mark.gpu
@pytest.mark.parametrize("fused,B,dtype,kind",
                         [(1, *c) for c in MOE_TIE_CASES] + [(0, *c) for c in MOE_TIE_CASES
                                                             if c[0] == 1])
def test_moe_block_probability_ties(gpu, fused, B, dtype, kind):
    """The MoE block's own routing (single-launch B=1, per-token and MFMA
    paths) on tie cases: indices bit-exact, output within tolerance."""
    import torch
    from logan_amd import _lib
    from logan_amd.device import moe_block

    from test_moe_gpu import Layer

    print(f"moe ties B={B} {dtype} {kind} fused={fused}", flush=True)
    _lib.lib().logan_hip_set_moe_fused(fused)
    try:
        layer = Layer(torch, E, K, 2048, 512, 4, 64, seed=77)
        rng = np.random.default_rng(78)
        xb = make_x(rng, B, 2048)
        lf = np.stack([tie_logits(kind, 100 + s) for s in range(B)])
        x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
        out, idx, w = moe_block(layer.dev, x, dev_logits(torch, lf, dtype), return_routing=True,
                                out_dtype=torch.float32)
        out, idx = out.cpu().numpy(), idx.cpu().numpy()
        xf = bf16_to_f32(xb)
        for t in range(B):
            ref, ridx, _ = layer.ref(xf[t], lf[t])
            np.testing.assert_array_equal(idx[t], ridx)
            if kind in NAN_KINDS:  # NaN weights: the reference's output is NaN throughout
                assert np.isnan(ref).all() and np.isnan(out[t]).all()
            else:
                assert normwise_rel(out[t], ref) <= 5e-5
    finally:
        _lib.lib().logan_hip_set_moe_fused(1)
    assert _lib.lib().logan_hip_moe_sync_errors() == 0
