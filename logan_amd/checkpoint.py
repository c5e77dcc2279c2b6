"""MLX quantized weights from safetensors checkpoints into HBM.

Host-side mirror of the reference loader for this path — `StFile`
(logan-qwen4/src/lib.rs:288-800), `load_mlx_quantized_wt` (:11818-11937) and
`load_mlx_quantized_expert_wt` (:11939-12078) — over the C ABI's layer 3
(include/logan_hip.h). Parsing, validation and the upload run in
liblogan_hip.so; a rejected tensor raises `CheckpointError` with the
reference's own message (its `Err(String)`).

The loaded objects speak the protocol of `device.AffineMatrix`,
`device.AffineBank` and `device.Mxfp4Matrix` (`.c()` plus geometry), so they
feed `device.affine_gemv`, `device.moe_block`, `device.mxfp4_gemv` directly.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, List, Optional

import numpy as np

from . import _lib as L

DTYPES = ("F32", "I32", "I64", "U32", "U8", "BF16", "F16", "F8_E4M3", "F8_E4M3FN")


class CheckpointError(RuntimeError):
    pass


def _err() -> str:
    m = L.lib().logan_hip_last_error()
    return m.decode() if m else "unknown error"


class StFile:
    """An open safetensors checkpoint (one file, or a sharded directory)."""

    def __init__(self, handle: int):
        self._h = handle

    @classmethod
    def open(cls, path) -> "StFile":
        h = L.lib().logan_hip_st_open(str(path).encode())
        if not h:
            raise CheckpointError(_err())
        return cls(h)

    @classmethod
    def open_dir(cls, path) -> "StFile":
        h = L.lib().logan_hip_st_open_dir(str(path).encode())
        if not h:
            raise CheckpointError(_err())
        return cls(h)

    def close(self) -> None:
        if self._h:
            L.lib().logan_hip_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def handle(self) -> int:
        if not self._h:
            raise CheckpointError("checkpoint is closed")
        return self._h

    def shard_count(self) -> int:
        return int(L.lib().logan_hip_st_shard_count(self.handle))

    def dtype_counts(self) -> Dict[str, int]:
        out = {}
        for d in DTYPES:
            n = int(L.lib().logan_hip_st_dtype_count(self.handle, d.encode()))
            if n:
                out[d] = n
        return out

    def _info(self, name: str):
        dt = C.create_string_buffer(32)
        shape = (C.c_uint64 * 16)()
        nd = C.c_int(0)
        nb = C.c_uint64(0)
        if not L.lib().logan_hip_st_tensor(self.handle, name.encode(), dt, 32, shape, 16,
                                           C.byref(nd), C.byref(nb)):
            return None
        return dt.value.decode(), [int(shape[i]) for i in range(min(nd.value, 16))], int(nb.value)

    def shape_of(self, name: str) -> Optional[List[int]]:
        i = self._info(name)
        return None if i is None else i[1]

    def dtype_of(self, name: str) -> Optional[str]:
        i = self._info(name)
        return None if i is None else i[0]

    def nbytes_of(self, name: str) -> Optional[int]:
        i = self._info(name)
        return None if i is None else i[2]

    def payload_range(self, name: str, within: int, length: int) -> bytes:
        buf = C.create_string_buffer(max(1, length))
        rc = L.lib().logan_hip_st_read(self.handle, name.encode(), within, length, buf)
        if rc != 1:
            raise CheckpointError(_err())
        return buf.raw[:length]

    def payload(self, name: str) -> bytes:
        n = self.nbytes_of(name)
        if n is None:
            raise CheckpointError(f"missing tensor {name}")
        return self.payload_range(name, 0, n)


class _Owned:
    """A LoganHipQuantWt and the device allocation behind it."""

    def __init__(self, q: L.QuantWt):
        self.q = q
        self.device = None
        try:
            import torch

            if torch.cuda.is_available():
                self.device = torch.device("cuda", torch.cuda.current_device())
        except ImportError:
            pass

    def __del__(self):
        try:
            if self.q.owner:
                L.lib().logan_hip_quant_free(C.byref(self.q))
        except Exception:
            pass


class LoadedAffine:
    """One MLX-affine matrix in HBM (expert `e` of a loaded bank, or a dense
    matrix): the protocol of device.AffineMatrix."""

    def __init__(self, own: _Owned, e: int = 0):
        q = own.q
        self._own = own
        self.device = own.device
        self.O, self.I, self.bits, self.group_size = q.O, q.I, q.bits, q.group_size
        self.aux_fp16 = bool(q.aux_fp16)
        wb = q.O * q.I * q.bits // 8
        pb = q.O * (q.I // q.group_size) * 2
        self.w_ptr = q.weights + e * wb
        self.sc_ptr = q.scales + e * pb
        self.bi_ptr = q.biases + e * pb

    def c(self) -> L.Affine:
        return L.Affine(self.w_ptr, self.sc_ptr, self.bi_ptr, self.O, self.I, self.bits,
                        self.group_size, int(self.aux_fp16))

    def as_bank(self) -> "LoadedAffineBank":
        """A dense matrix as a one-expert bank (a shared expert's slot)."""
        if self._own.q.E != 1:
            raise CheckpointError("only a dense matrix is a one-expert bank")
        return LoadedAffineBank(self._own)


class LoadedAffineBank:
    """E stacked experts (switch_mlp) in HBM: the protocol of
    device.AffineBank."""

    def __init__(self, own: _Owned):
        q = own.q
        self._own = own
        self.device = own.device
        self.E, self.O, self.I, self.bits = q.E, q.O, q.I, q.bits
        self.group_size, self.aux_fp16 = q.group_size, bool(q.aux_fp16)

    def c(self) -> L.AffineBank:
        q = self._own.q
        return L.AffineBank(q.weights, q.scales, q.biases, q.E, q.O, q.I, q.bits, q.group_size,
                            q.aux_fp16)

    def expert(self, e: int) -> LoadedAffine:
        if not 0 <= e < self.E:
            raise IndexError(e)
        return LoadedAffine(self._own, e)


class LoadedMxfp4:
    """One MXFP4 matrix in HBM (expert `e` of a loaded stack, or dense): the
    protocol of device.Mxfp4Matrix (one plane)."""

    def __init__(self, own: _Owned, e: int = 0):
        q = own.q
        self._own = own
        self.device = own.device
        self.O, self.I, self.planes = q.O, q.I, 1
        self.codes_ptr = q.weights + e * q.O * (q.I // 2)
        self.scales_ptr = q.scales + e * q.O * ((q.I + 31) // 32)

    def c(self) -> L.Mxfp4:
        return L.Mxfp4(self.codes_ptr, self.scales_ptr, self.O, self.I, 1)


class LoadedMxfp4Stack:
    def __init__(self, own: _Owned):
        self._own = own
        self.E, self.O, self.I = own.q.E, own.q.O, own.q.I

    def expert(self, e: int) -> LoadedMxfp4:
        if not 0 <= e < self.E:
            raise IndexError(e)
        return LoadedMxfp4(self._own, e)


def _wrap(q: L.QuantWt, bank: bool):
    own = _Owned(q)
    if q.kind == L.LOGAN_HIP_WT_AFFINE:
        return LoadedAffineBank(own) if bank else LoadedAffine(own)
    return LoadedMxfp4Stack(own) if bank else LoadedMxfp4(own)


def plan_mlx_quantized_wt(st: StFile, name: str, o: int, i: int) -> L.QuantWt:
    """load_mlx_quantized_wt's checks only (nothing read or allocated)."""
    q = L.QuantWt()
    if L.lib().logan_hip_plan_mlx_quantized(st.handle, name.encode(), o, i, C.byref(q)) != 1:
        raise CheckpointError(_err())
    return q


def plan_mlx_quantized_experts(st: StFile, name: str, e0: int, count: int, experts: int, o: int,
                               i: int) -> L.QuantWt:
    q = L.QuantWt()
    if L.lib().logan_hip_plan_mlx_quantized_experts(st.handle, name.encode(), e0, count, experts,
                                                    o, i, C.byref(q)) != 1:
        raise CheckpointError(_err())
    return q


def load_mlx_quantized_wt(st: StFile, name: str, o: int, i: int):
    """A dense packed matrix `name` (U32 [o, words]) into HBM
    (logan-qwen4/src/lib.rs:11818-11937): LoadedAffine or LoadedMxfp4."""
    q = L.QuantWt()
    rc = L.lib().logan_hip_load_mlx_quantized(st.handle, name.encode(), o, i, C.byref(q))
    if rc != 1:
        raise CheckpointError(_err())
    return _wrap(q, bank=False)


def load_mlx_quantized_expert_wt(st: StFile, name: str, expert: int, experts: int, o: int,
                                 i: int):
    """One expert's slice of a stacked switch_mlp bank into HBM
    (lib.rs:11939-12078): LoadedAffine or LoadedMxfp4."""
    q = L.QuantWt()
    rc = L.lib().logan_hip_load_mlx_quantized_experts(st.handle, name.encode(), expert, 1,
                                                      experts, o, i, C.byref(q))
    if rc != 1:
        raise CheckpointError(_err())
    return _wrap(q, bank=False)


def load_mlx_quantized_bank(st: StFile, name: str, experts: int, o: int, i: int, e0: int = 0,
                            count: Optional[int] = None):
    """Experts [e0, e0 + count) of a stacked bank (all of them by default)
    resident in one transfer: LoadedAffineBank or LoadedMxfp4Stack."""
    n = experts - e0 if count is None else count
    q = L.QuantWt()
    rc = L.lib().logan_hip_load_mlx_quantized_experts(st.handle, name.encode(), e0, n, experts,
                                                      o, i, C.byref(q))
    if rc != 1:
        raise CheckpointError(_err())
    return _wrap(q, bank=True)


class CachedBankGeometry:
    """A routed bank whose experts live in an ExpertCache: only its geometry
    (the protocol of device.AffineBank's c(), weight pointers null)."""

    def __init__(self, E: int, O: int, I: int, bits: int, group_size: int, aux_fp16: bool = False):
        self.E, self.O, self.I, self.bits = E, O, I, bits
        self.group_size, self.aux_fp16 = group_size, aux_fp16

    def c(self) -> L.AffineBank:
        return L.AffineBank(None, None, None, self.E, self.O, self.I, self.bits, self.group_size,
                            int(self.aux_fp16))


class ExpertCache:
    """The reference's route-driven expert cache and route arena
    (RouteCache / RouteArena, logan-qwen4/src/lib.rs:12110-12300,
    cache_fetch_route :12697-12903) in HBM, filled from this checkpoint
    (logan_hip_expert_cache_*): `fetch` places one token's routed experts and
    returns their blocks for device.moe_block_cached."""

    def __init__(self, st: StFile, experts: int, d_model: int, d_hidden: int,
                 blocks_per_layer: int, topk: int, layers: int = 0):
        self._st = st  # the cache reads the checkpoint's descriptors: keep it open
        self.experts, self.d_model, self.d_hidden = experts, d_model, d_hidden
        h = L.lib().logan_hip_expert_cache_create(st.handle, layers, experts, d_model, d_hidden,
                                                  blocks_per_layer, topk)
        if not h:
            raise CheckpointError(_err())
        self._h = h
        s = self.stats()
        self.layers, self.blocks_per_layer, self.topk = s["layers"], s["blocks_per_layer"], s["topk"]

    @property
    def handle(self) -> int:
        if not self._h:
            raise CheckpointError("expert cache is closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            L.lib().logan_hip_expert_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def fetch(self, layer: int, experts, stream=None) -> np.ndarray:
        """Blocks of the route's experts (rank order); loads the misses and the
        arena ranks, ordered after `stream`'s queued work, and makes `stream`
        wait for them. None when the cache declines the route."""
        e = np.ascontiguousarray(experts, dtype=np.int32)
        blocks = np.empty(len(e), np.int32)
        st = None
        if stream is not None:
            st = stream.cuda_stream or None
        else:
            try:
                import torch

                if torch.cuda.is_available():
                    st = torch.cuda.current_stream().cuda_stream or None
            except ImportError:
                pass
        rc = L.lib().logan_hip_expert_cache_fetch(self.handle, layer, e.ctypes.data, len(e),
                                                  blocks.ctypes.data, st)
        if rc == 0:
            return None
        if rc != 1:
            raise CheckpointError(_err())
        return blocks

    def stats(self) -> Dict[str, int]:
        s = L.ExpertCacheStats()
        L.lib().logan_hip_expert_cache_stats(self.handle, C.byref(s))
        return {name: int(getattr(s, name)) for name, _ in L.ExpertCacheStats._fields_}

    def tags(self, layer: int) -> np.ndarray:
        out = np.empty(max(self.blocks_per_layer, 1), np.int32)
        if L.lib().logan_hip_expert_cache_tags(self.handle, layer, out.ctypes.data) != 1:
            raise CheckpointError("bad layer")
        return out[:self.blocks_per_layer]

    def geometry(self, bits: int, group_size: int, aux_fp16: bool = False, down_group_size=None):
        """(gate, up, down) CachedBankGeometry for a device.MoeLayer."""
        dg = group_size if down_group_size is None else down_group_size
        return (CachedBankGeometry(self.experts, self.d_hidden, self.d_model, bits, group_size, aux_fp16),
                CachedBankGeometry(self.experts, self.d_hidden, self.d_model, bits, group_size, aux_fp16),
                CachedBankGeometry(self.experts, self.d_model, self.d_hidden, bits, dg, aux_fp16))
