"""Test helpers independent of the oracle: an MLX packer written from the
format statement (LSB-first bitstream of little-endian u32 words,
logan-qwen4/src/colisource.rs:719-722) with numpy bit arrays, float64
dequantisation, and the reference's error metrics."""
from __future__ import annotations

import numpy as np

from logan_amd.synth import bf16_bits, bf16_to_f32


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """codes [O, I] (ints < 2^bits) -> packed bytes [O, I*bits/8]."""
    codes = np.asarray(codes, dtype=np.uint64)
    O, I = codes.shape
    assert (I * bits) % 32 == 0
    bitarr = ((codes[:, :, None] >> np.arange(bits, dtype=np.uint64)) & 1).astype(np.uint8)
    return np.packbits(bitarr.reshape(O, I * bits), axis=1, bitorder="little")


def unpack_codes(packed: np.ndarray, I: int, bits: int) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    O = packed.shape[0]
    bitarr = np.unpackbits(packed, axis=1, bitorder="little")[:, : I * bits]
    bitarr = bitarr.reshape(O, I, bits).astype(np.uint64)
    return (bitarr << np.arange(bits, dtype=np.uint64)).sum(axis=2)


def params_f32(p: np.ndarray, fp16: bool) -> np.ndarray:
    p = np.asarray(p, dtype=np.uint16)
    return p.view(np.float16).astype(np.float32) if fp16 else bf16_to_f32(p)


def dequant_f64(packed, sc, bi, O, I, bits, gs, fp16=False) -> np.ndarray:
    codes = unpack_codes(np.asarray(packed).reshape(O, -1), I, bits).astype(np.float64)
    s = np.repeat(params_f32(sc, fp16).reshape(O, I // gs).astype(np.float64), gs, axis=1)
    b = np.repeat(params_f32(bi, fp16).reshape(O, I // gs).astype(np.float64), gs, axis=1)
    return codes * s + b


def normwise_rel(got, want) -> float:
    """max|got-want| / max|want| (the reference's convention,
    logan-qwen4/src/lib.rs:17164-17173)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-6)
    return float(np.abs(got - want).max() / scale)


def bf16_ulp_ok(got_bits: np.ndarray, want_f32: np.ndarray, ulps: int = 1) -> bool:
    """bf16 output within `ulps` of RNE(fp32 reference), compared as ordered
    integers."""
    def ordered(b):
        b = np.asarray(b, np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    g = ordered(np.asarray(got_bits, np.uint16).astype(np.int32))
    w = ordered(bf16_bits(np.asarray(want_f32, np.float32)).astype(np.int32))
    return bool(np.all(np.abs(g - w) <= ulps))


__all__ = ["pack_codes", "unpack_codes", "dequant_f64", "normwise_rel", "bf16_ulp_ok",
           "params_f32", "bf16_bits", "bf16_to_f32"]
