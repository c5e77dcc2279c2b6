"""Seeded synthetic inputs in the benchmark's data scheme.

* packed codes: uniform random u32 words, so every b-bit code (including codes
  that straddle words) is uniform on [0, 2^b - 1];
* scale = bf16(|N(0,1)| * 0.01), bias = -2^(b-1) * scale (exact in bf16/fp16;
  for 4-bit this is the -8*scale of the 4-bit configuration);
* activations and router logits: bf16(N(0,1));
* Zipf-skewed router logits: bf16(-s*ln(rank_e) + Gumbel(0,1)) with a seeded
  random rank per expert, so the top-1 expert is distributed exactly as
  Zipf(s) (Gumbel-max) and the top-k follow the same popularity.
"""
from __future__ import annotations

import numpy as np


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (logan-core/src/math.rs:279-283)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_params(rng: np.random.Generator, shape, bits: int, fp16: bool = False):
    """(scales, biases) as u16 bit arrays of `shape`."""
    sc = np.abs(rng.standard_normal(shape, dtype=np.float32)) * np.float32(0.01)
    if fp16:
        s16 = sc.astype(np.float16)
        b16 = (s16.astype(np.float32) * np.float32(-(2 ** (bits - 1)))).astype(np.float16)
        return s16.view(np.uint16), b16.view(np.uint16)
    s = bf16_bits(sc)
    b = bf16_bits(bf16_to_f32(s) * np.float32(-(2 ** (bits - 1))))
    return s, b


def make_affine(rng: np.random.Generator, O: int, I: int, bits: int, gs: int,
                fp16: bool = False, E: int | None = None):
    """Packed weights (u8 [.., O, I*bits/8]) plus scales/biases (u16 [.., O, I/gs])."""
    lead = () if E is None else (E,)
    words = rng.integers(0, 2 ** 32, size=lead + (O, I * bits // 32), dtype=np.uint32)
    sc, bi = make_params(rng, lead + (O, I // gs), bits, fp16)
    w = words.view(np.uint8).reshape(lead + (O, I * bits // 8))
    return w, sc, bi


def make_x(rng: np.random.Generator, *shape) -> np.ndarray:
    return bf16_bits(rng.standard_normal(shape, dtype=np.float32))


def make_logits(rng: np.random.Generator, B: int, E: int, zipf_s: float | None = None) -> np.ndarray:
    if zipf_s is None:
        return bf16_bits(rng.standard_normal((B, E), dtype=np.float32))
    rank = rng.permutation(E).astype(np.float64) + 1.0
    prior = -zipf_s * np.log(rank)
    gumbel = -np.log(-np.log(rng.uniform(1e-12, 1.0, size=(B, E))))
    return bf16_bits((prior[None, :] + gumbel).astype(np.float32))


def aux_bytes(sc: np.ndarray, bi: np.ndarray) -> np.ndarray:
    """The reference's combined sidecar: all scales, then all biases
    (backend_metal.mm:218-220)."""
    return np.concatenate([sc.reshape(-1), bi.reshape(-1)]).view(np.uint8)


# ---------------------------------------------------------------- device side

def torch_affine(O: int, I: int, bits: int, gs: int, E: int | None = None, seed: int = 0,
                 device: str = "cuda"):
    """Same scheme generated directly in HBM (for benchmark-sized banks)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    lead = () if E is None else (E,)
    words = torch.randint(-(2 ** 31), 2 ** 31, lead + (O, I * bits // 32), dtype=torch.int32,
                          device=device, generator=g)
    w = words.view(torch.uint8).reshape(lead + (O, I * bits // 8))
    sc = (torch.randn(lead + (O, I // gs), device=device, generator=g).abs() * 0.01).to(torch.bfloat16)
    bi = (sc.float() * -(2 ** (bits - 1))).to(torch.bfloat16)
    return w, sc.view(torch.int16), bi.view(torch.int16)
