"""CPU oracle for the logan-hip hot path — TEST INFRASTRUCTURE ONLY.

ctypes wrapper over liblogan_oracle.so (oracle/oracle.c), a plain-C
restatement of the reference's CPU arithmetic (each C function cites the
reference file:line it follows). Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this module, and only as the checker
or the reported CPU baseline; the library (logan_amd) never uses it.

Pinning (tests/test_oracle.py): every function is checked against the
reference's own known-answer vectors (tests/golden/kat_vectors.json, taken
from the reference tests cited there) and against independent arithmetic
(numpy unpacking, float64 matmuls, exhaustive fp16 decoding, stable-argsort
top-k, closed forms). No function is "parity unpinned".
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SO = HERE / "liblogan_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return SO


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not SO.exists():
            build()
        h = C.CDLL(str(SO))
        P, SZ, I = C.c_void_p, C.c_size_t, C.c_int
        h.lo_f16_to_f32.restype = C.c_float
        h.lo_f16_to_f32.argtypes = [C.c_uint16]
        h.lo_f32_to_bf16.restype = C.c_uint16
        h.lo_f32_to_bf16.argtypes = [C.c_float]
        h.lo_bf16_to_f32.restype = C.c_float
        h.lo_bf16_to_f32.argtypes = [C.c_uint16]
        h.lo_affine_code.restype = C.c_uint32
        h.lo_affine_code.argtypes = [P, SZ, I]
        h.lo_affine_param.restype = C.c_float
        h.lo_affine_param.argtypes = [P, SZ, I]
        h.lo_affine_dequant.restype = I
        h.lo_affine_dequant.argtypes = [P, P, P, P, SZ, SZ, I, SZ, I, SZ, SZ]
        h.lo_affine_gemv.restype = None
        h.lo_affine_gemv.argtypes = [P, P, P, P, P, SZ, SZ, I, SZ, I]
        h.lo_affine_gemv_mt.restype = None
        h.lo_affine_gemv_mt.argtypes = [P, P, P, P, P, SZ, SZ, I, SZ, I, I]
        h.lo_spark_affine8_gemv.restype = None
        h.lo_spark_affine8_gemv.argtypes = [P, P, P, P, SZ, SZ]
        h.lo_affine_qmm_bf16.restype = None
        h.lo_affine_qmm_bf16.argtypes = [P, P, P, P, P, SZ, SZ, SZ, I, SZ, I]
        h.lo_mxfp4_value.restype = C.c_float
        h.lo_mxfp4_value.argtypes = [C.c_uint8, C.c_uint8]
        h.lo_mxfp4_gemv_stacked.restype = None
        h.lo_mxfp4_gemv_stacked.argtypes = [P, P, P, P, SZ, SZ, I]
        h.lo_dense_gemv.restype = None
        h.lo_dense_gemv.argtypes = [P, P, P, P, P, I, SZ, SZ]
        h.lo_llama_layer.restype = I
        h.lo_llama_layer.argtypes = [P, P, P, I, P, P, P, P, P, P, I, I, I, I, I, C.c_float,
                                     C.c_float]
        h.lo_rmsnorm.restype = None
        h.lo_rmsnorm.argtypes = [P, P, SZ, SZ, C.c_float]
        h.lo_add.restype = None
        h.lo_add.argtypes = [P, P, SZ]
        h.lo_silu.restype = C.c_float
        h.lo_silu.argtypes = [C.c_float]
        h.lo_silu_mul.restype = None
        h.lo_silu_mul.argtypes = [P, P, SZ]
        h.lo_softmax_row.restype = None
        h.lo_softmax_row.argtypes = [P, SZ]
        h.lo_topk.restype = C.c_float
        h.lo_topk.argtypes = [P, SZ, SZ, P, P]
        h.lo_moe_token.restype = None
        h.lo_moe_token.argtypes = [P, P, P, SZ, SZ, SZ, P, P, P, P, P, P, P, P, P]
        h.lo_moe_token_mt.restype = None
        h.lo_moe_token_mt.argtypes = [P, P, P, SZ, SZ, SZ, P, P, P, P, P, P, P, P, P, I]
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def threads() -> int:
    return int(os.environ.get("LOGAN_ORACLE_THREADS", min(8, os.cpu_count() or 1)))


def affine_code(row: np.ndarray, column: int, bits: int) -> int:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    return int(lib().lo_affine_code(_p(row), column, bits))


def affine_dequant(w, sc, bi, rows, cols, bits, gs, fp16=False, row0=0, nrows=None) -> np.ndarray:
    n = rows - row0 if nrows is None else nrows
    out = np.empty((n, cols), np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(sc).view(np.uint8)
    bi = np.ascontiguousarray(bi).view(np.uint8)
    rc = lib().lo_affine_dequant(_p(out), _p(w), _p(sc), _p(bi), rows, cols, bits, gs, int(fp16),
                                 row0, n)
    if rc != 0:
        raise ValueError("invalid affine geometry")
    return out


def affine_gemv(x: np.ndarray, w, sc, bi, O, I, bits, gs, fp16=False, nthreads=None) -> np.ndarray:
    """y = W x for one f32 activation row (logan-qwen4/src/lib.rs:3729-3764)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(O, np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(sc).view(np.uint8)
    bi = np.ascontiguousarray(bi).view(np.uint8)
    t = threads() if nthreads is None else nthreads
    if t <= 1:
        lib().lo_affine_gemv(_p(y), _p(x), _p(w), _p(sc), _p(bi), O, I, bits, gs, int(fp16))
    else:
        lib().lo_affine_gemv_mt(_p(y), _p(x), _p(w), _p(sc), _p(bi), O, I, bits, gs, int(fp16), t)
    return y


def affine_qmm_bf16(x: np.ndarray, w, sc, bi, O, I, bits, gs, fp16=False) -> np.ndarray:
    """Y[M, O] = X[M, I] . bf16(W)^T, f32 accumulation
    (logan-metal/metal/backend_metal.mm:1480-1560)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, I)
    M = x.shape[0]
    y = np.empty((M, O), np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(sc).view(np.uint8)
    bi = np.ascontiguousarray(bi).view(np.uint8)
    lib().lo_affine_qmm_bf16(_p(y), _p(x), _p(w), _p(sc), _p(bi), M, O, I, bits, gs, int(fp16))
    return y


def spark_affine8_gemv(x, w, aux, O, I) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(O, np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    aux = np.ascontiguousarray(aux).view(np.uint8)
    lib().lo_spark_affine8_gemv(_p(y), _p(x), _p(w), _p(aux), O, I)
    return y


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(g) * u element-wise in f32 (returns a new array)."""
    out = np.ascontiguousarray(g, np.float32).copy()
    uu = np.ascontiguousarray(u, np.float32)
    assert out.size == uu.size
    lib().lo_silu_mul(_p(out), _p(uu), out.size)
    return out


def mxfp4_value(code: int, scale_byte: int) -> float:
    return float(lib().lo_mxfp4_value(code, scale_byte))


def mxfp4_gemv(x: np.ndarray, w, sc, O: int, I: int, stacks: int = 1) -> np.ndarray:
    """y = W x for MXFP4 weights (fmt 7; stacks 2 / 3 = fmt 9 / 10):
    w u8 [stacks][O][I/2], sc u8 [stacks][O][I/32]
    (logan-qwen4/src/lib.rs:2932-3038)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(sc, np.uint8)
    assert w.size >= stacks * O * ((I + 1) // 2) and sc.size >= stacks * O * ((I + 31) // 32)
    y = np.empty(O, np.float32)
    lib().lo_mxfp4_gemv_stacked(_p(y), _p(x), _p(w), _p(sc), O, I, stacks)
    return y


def dense_gemv(x: np.ndarray, w, O: int, I: int, fmt: int, sc=None, bi=None) -> np.ndarray:
    """y = W x for bf16-valued weights: fmt 5 w = bf16 bits u16 [O, I]; fmt 15
    w = affine-8 codes u8 [O, I] with bf16 scale/bias bits [O, I/64]
    (logan-llama/src/model.rs:1025-1033, weights.rs:441-516)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w)
    y = np.empty(O, np.float32)
    scp = np.ascontiguousarray(sc, np.uint16) if fmt == 15 else None
    bip = np.ascontiguousarray(bi, np.uint16) if fmt == 15 else None
    lib().lo_dense_gemv(_p(y), _p(x), _p(w), _p(scp) if scp is not None else None,
                        _p(bip) if bip is not None else None, fmt, O, I)
    return y


def llama_layer(x, kc, vc, pos: int, mats, in_norm, post_norm, D, inter, H, KH, hd, theta, eps):
    """One decode layer (logan-llama/src/model.rs:786-905). x [D] f32 (a new
    array is returned); kc / vc [>= pos+1, KH*hd] f32 are updated in place at
    row pos. mats: 7 tuples (fmt, w, sc, bi) for q, k, v, o, gate, up, down."""
    out = np.array(x, np.float32, copy=True)
    assert kc.dtype == np.float32 and vc.dtype == np.float32
    assert kc.flags.c_contiguous and vc.flags.c_contiguous
    keep = []
    W, S, B, F = (C.c_void_p * 7)(), (C.c_void_p * 7)(), (C.c_void_p * 7)(), (C.c_int * 7)()
    for i, (fmt, w, sc, bi) in enumerate(mats):
        w = np.ascontiguousarray(w)
        keep.append(w)
        W[i] = w.ctypes.data
        F[i] = fmt
        if fmt == 15:
            sc = np.ascontiguousarray(sc, np.uint16)
            bi = np.ascontiguousarray(bi, np.uint16)
            keep += [sc, bi]
            S[i], B[i] = sc.ctypes.data, bi.ctypes.data
    inn = np.ascontiguousarray(in_norm, np.float32)
    pon = np.ascontiguousarray(post_norm, np.float32)
    rc = lib().lo_llama_layer(_p(out), _p(kc), _p(vc), pos, W, S, B, F, _p(inn), _p(pon), D, inter,
                              H, KH, hd, theta, eps)
    assert rc == 1
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Row-wise x * (1/sqrt(mean(x^2) + eps)) * w of x [nrows, n] (new array)."""
    out = np.array(x, np.float32, copy=True, order="C")
    ww = np.ascontiguousarray(w, np.float32)
    n = ww.size
    assert out.size % n == 0
    lib().lo_rmsnorm(_p(out), _p(ww), n, out.size // n, eps)
    return out


def add(y: np.ndarray, a: np.ndarray) -> np.ndarray:
    out = np.array(y, np.float32, copy=True, order="C")
    aa = np.ascontiguousarray(a, np.float32)
    assert out.size == aa.size
    lib().lo_add(_p(out), _p(aa), out.size)
    return out


def softmax_row(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().lo_softmax_row(_p(y), y.size)
    return y


def topk(probs: np.ndarray, k: int):
    probs = np.ascontiguousarray(probs, np.float32)
    idx = np.empty(k, np.int32)
    val = np.empty(k, np.float32)
    wsum = lib().lo_topk(_p(probs), probs.size, k, _p(idx), _p(val))
    return idx, val, float(wsum)


class Bank(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("o", C.c_size_t), ("i", C.c_size_t), ("bits", C.c_int),
                ("group_size", C.c_size_t), ("fp16", C.c_int)]


def _bank(w, sc, bi, O, I, bits, gs, fp16, keep):
    w = np.ascontiguousarray(w, np.uint8)
    sc = np.ascontiguousarray(sc).view(np.uint8)
    bi = np.ascontiguousarray(bi).view(np.uint8)
    b = Bank(_p(w), _p(sc), _p(bi), O, I, bits, gs, int(fp16))
    keep += [w, sc, bi, b]
    return C.addressof(b)


def moe_token(x, logits, k, D, inter, bits, gs, gate, up, down, shared=None, se_g=None,
              sinter=None, fp16=False, nthreads=None):
    """One token of the routed-MoE block. gate/up/down are (w, sc, bi) of
    stacked banks; shared is (gate, up, down) of single experts (or None).
    Returns (out[D], idx[k], w[k])."""
    keep = []
    x = np.ascontiguousarray(x, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    E = logits.size
    g = _bank(*gate, inter, D, bits, gs, fp16, keep)
    u = _bank(*up, inter, D, bits, gs, fp16, keep)
    dn = _bank(*down, D, inter, bits, gs, fp16, keep)
    out = np.empty(D, np.float32)
    idx = np.empty(k, np.int32)
    wt = np.empty(k, np.float32)
    sp = [None, None, None]
    seg = None
    if shared is not None:
        si = inter if sinter is None else sinter
        sp = [_bank(*shared[0], si, D, bits, gs, fp16, keep),
              _bank(*shared[1], si, D, bits, gs, fp16, keep),
              _bank(*shared[2], D, si, bits, gs, fp16, keep)]
        seg = np.ascontiguousarray(se_g, np.float32)
        keep.append(seg)
    t = threads() if nthreads is None else nthreads
    args = [_p(out), _p(x), _p(logits), E, k, D, g, u, dn,
            sp[0], sp[1], sp[2], _p(seg) if seg is not None else None, _p(idx), _p(wt)]
    if t <= 1:
        lib().lo_moe_token(*args)
    else:
        lib().lo_moe_token_mt(*args, t)
    return out, idx, wt
