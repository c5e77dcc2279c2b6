"""Host-side mirror of logan-metal's backend-neutral Rust surface, over the C ABI.

Same names and argument meaning as logan-metal/src/lib.rs, with `metal_`
replaced by `hip_` where the reference name carries the backend:

    metal_init / metal_available            :757-770   -> hip_init / hip_available
    metal_matmul (fmt 15, Spark)            :795-854   -> hip_matmul
    metal_matmul_mlx_affine                 :950-975   -> hip_matmul_mlx_affine
    metal_matmul_mlx_affine_multi           :977-1062  -> hip_matmul_mlx_affine_multi
    moe_route_begin / moe_route_finish      :3822-3883 -> moe_route_begin / moe_route_finish
    MoeRoutePending (Drop => discard)       :3803-3815 -> MoeRoutePending (close/__del__)
    shared_mxfp4 (MetalWeightDesc :188-196) :2583-2678 -> shared_mxfp4
    shared_mxfp4 (affine descriptors)                  -> shared_expert
    dense_profile_start / _stop             :772-789   -> dense_profile_start / _stop
    llama_layer / llama_drop_model          :1559-1681 -> llama_layer / llama_drop_model

Host arrays are numpy (f32 activations/outputs, u8 packed weights and the
[scales][biases] u16 sidecar as bytes). Validation declines (returns False /
None) exactly where the reference's wrappers do (:888-948, :977-1062,
:3822-3849). Tensor handles are plain ints kept by the caller in `Tensor`.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib as L


def hip_init() -> bool:
    return L.lib().logan_hip_init() == 1


def hip_available() -> bool:
    return L.lib().logan_hip_available() == 1


def mlx_affine_fmt(bits: int, aux_fp16: bool) -> Optional[int]:
    """logan-metal/src/lib.rs:860-880 (the Q4-FMA fmt 20 computes the same
    product, so the plain code 16 is used)."""
    table = {4: 0, 5: 1, 6: 2, 8: 3}
    if bits not in table:
        return None
    return (21 if aux_fp16 else 16) + table[bits]


@dataclass
class Tensor:
    """Caller-owned slot for the lazily created device handle
    (`Mutex<usize>` in the reference, logan-qwen4/src/lib.rs:1576-1577)."""

    handle: int = 0

    def free(self) -> None:
        if self.handle:
            L.lib().logan_hip_tensor_free(C.c_void_p(self.handle))
            self.handle = 0

    def nbytes(self) -> int:
        return int(L.lib().logan_hip_tensor_bytes(C.c_void_p(self.handle))) if self.handle else 0


def _f32(a: np.ndarray) -> np.ndarray:
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError("expected a C-contiguous float32 array")
    return a


def _bytes(a) -> np.ndarray:
    a = np.asarray(a)
    if not a.flags.c_contiguous:
        raise TypeError("expected a C-contiguous array")
    return a.view(np.uint8).reshape(-1)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def hip_matmul(tensor: Tensor, y: np.ndarray, x: np.ndarray, weights, scales, fmt: int,
               i: int, o: int, gs: int = 0, s: int = 1) -> bool:
    """logan-metal/src/lib.rs:795-854 (coli_metal_matmul, any fmt; this
    backend serves 15..24 and declines the rest)."""
    if not hip_available() or i <= 0 or o <= 0 or s <= 0:
        return False
    y, x = _f32(y), _f32(x)
    if x.size < s * i or y.size < s * o:
        return False
    w, a = _bytes(weights), _bytes(scales)
    h = C.c_void_p(tensor.handle or None)
    rc = L.lib().logan_hip_matmul(C.byref(h), _ptr(y), _ptr(x), _ptr(w), _ptr(a), fmt, s, i, o, gs)
    tensor.handle = h.value or 0
    return rc == 1


def _affine_geometry_ok(bits: int, group_size: int, aux_fp16: bool, i: int, o: int,
                        weights: np.ndarray, aux: np.ndarray) -> Optional[int]:
    """Rust-side validation of logan-metal/src/lib.rs:901-933; returns fmt."""
    if i == 0 or o == 0 or group_size == 0 or i % group_size != 0:
        return None
    fmt = mlx_affine_fmt(bits, aux_fp16)
    if fmt is None:
        return None
    row_bits = i * bits
    if row_bits % 32 != 0:
        return None
    if weights.size < o * (row_bits // 8):
        return None
    if aux.size < 2 * o * (i // group_size) * 2:
        return None
    return fmt


def hip_matmul_mlx_affine(tensor: Tensor, y: np.ndarray, x: np.ndarray, weights, aux, bits: int,
                          group_size: int, aux_fp16: bool, i: int, o: int) -> bool:
    """logan-metal/src/lib.rs:888-975."""
    if not hip_available():
        return False
    y, x = _f32(y), _f32(x)
    if x.size < i or y.size < o:
        return False
    w, a = _bytes(weights), _bytes(aux)
    fmt = _affine_geometry_ok(bits, group_size, aux_fp16, i, o, w, a)
    if fmt is None:
        return False
    h = C.c_void_p(tensor.handle or None)
    rc = L.lib().logan_hip_matmul(C.byref(h), _ptr(y), _ptr(x), _ptr(w), _ptr(a), fmt, 1, i, o,
                                  group_size)
    tensor.handle = h.value or 0
    return rc == 1


@dataclass
class MlxAffineMatmulDesc:
    """logan-metal/src/lib.rs:170-186."""

    tensor: Tensor
    y: np.ndarray
    weights: np.ndarray
    aux: np.ndarray
    bits: int
    group_size: int
    aux_fp16: bool
    i: int
    o: int
    x: Optional[np.ndarray] = None


@dataclass
class MetalWeightDesc:
    """logan-metal/src/lib.rs:188-196: one weight of any fmt the backend
    serves (7 / 9 / 10 MXFP4 with one / two / three planes, 15..24 affine);
    `scales` holds the E8M0 bytes (MXFP4) or the [scales][biases] sidecar."""

    tensor: Tensor
    weights: np.ndarray
    scales: np.ndarray
    fmt: int
    group_size: int
    i: int
    o: int
    y: Optional[np.ndarray] = None
    x: Optional[np.ndarray] = None


MXFP4_PLANES = {7: 1, 9: 2, 10: 3}


def _weight_desc_fmt(d: MetalWeightDesc, w: np.ndarray, a: np.ndarray) -> Optional[int]:
    """Byte-size checks by format, as lib.rs:2606-2640 makes them (MXFP4:
    ceil(i/2) code bytes and ceil(i/32) scale bytes per row and plane)."""
    if d.i <= 0 or d.o <= 0:
        return None
    planes = MXFP4_PLANES.get(d.fmt)
    if planes is not None:
        if w.size < planes * d.o * ((d.i + 1) // 2) or a.size < planes * d.o * ((d.i + 31) // 32):
            return None
        return d.fmt
    bits = {15: 8, 16: 4, 17: 5, 18: 6, 19: 8, 20: 4, 21: 4, 22: 5, 23: 6, 24: 8}.get(d.fmt)
    if bits is None:
        return None
    gs = 64 if d.fmt == 15 else d.group_size
    if gs <= 0 or d.i % gs != 0:
        return None
    if w.size < d.o * ((d.i * bits + 7) // 8) or a.size < 2 * d.o * (d.i // gs) * 2:
        return None
    return d.fmt


def _raw_descs(descs, with_y: bool):
    raw = (L.MatmulDesc * len(descs))()
    keep = []
    for k, d in enumerate(descs):
        if isinstance(d, MetalWeightDesc):
            w, a = _bytes(d.weights), _bytes(d.scales)
            fmt = _weight_desc_fmt(d, w, a)
        else:
            w, a = _bytes(d.weights), _bytes(d.aux)
            fmt = _affine_geometry_ok(d.bits, d.group_size, d.aux_fp16, d.i, d.o, w, a)
        if fmt is None:
            return None, None
        if with_y:
            y = _f32(d.y)
            if y.size < d.o:
                return None, None
            raw[k].y = _ptr(y)
        if d.x is not None:
            x = _f32(d.x)
            if x.size < d.i:
                return None, None
            raw[k].x = _ptr(x)
            raw[k].S = 1
            keep.append(x)
        else:
            raw[k].x = None
            raw[k].S = 1
        raw[k].tensor = d.tensor.handle or None
        raw[k].weights = _ptr(w)
        raw[k].scales = _ptr(a)
        raw[k].fmt = fmt
        raw[k].I = d.i
        raw[k].O = d.o
        raw[k].gs = 0 if fmt in MXFP4_PLANES else d.group_size
        keep += [w, a]
    return raw, keep


def _write_back(descs, raw) -> None:
    for d, r in zip(descs, raw):
        d.tensor.handle = r.tensor or 0


def hip_matmul_mlx_affine_multi(x: np.ndarray, descs: Sequence[MlxAffineMatmulDesc]) -> bool:
    """logan-metal/src/lib.rs:977-1062: up to 16 descriptors, one submission."""
    if not hip_available() or not descs or len(descs) > 16:
        return False
    x = _f32(x) if x is not None and x.size else np.zeros(0, np.float32)
    for d in descs:
        if d.x is None and x.size < d.i:
            return False
    raw, keep = _raw_descs(descs, with_y=True)
    if raw is None:
        return False
    rc = L.lib().logan_hip_matmul_multi(_ptr(x) if x.size else None, 1, raw, len(descs))
    _write_back(descs, raw)
    return rc == 1


class MoeRoutePending:
    """Owning handle of one submitted route island (logan-metal/src/lib.rs:3803-3815)."""

    def __init__(self, raw: int, k: int, d: int):
        self.raw, self.k, self.d = raw, k, d

    def close(self) -> None:
        if self.raw:
            L.lib().logan_hip_moe_route_discard(C.c_void_p(self.raw))
            self.raw = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def moe_route_begin(descs: Sequence[MlxAffineMatmulDesc], x: np.ndarray, d: int,
                    m: int) -> Optional[MoeRoutePending]:
    """logan-metal/src/lib.rs:3822-3871: descs are K*3, expert-major
    [gate, up, down]; None is the pre-submit decline."""
    if not hip_available() or not descs or len(descs) % 3 != 0:
        return None
    x = _f32(x)
    if x.size < d:
        return None
    k = len(descs) // 3
    if k == 0 or k > 16:
        return None
    raw, keep = _raw_descs(descs, with_y=False)
    if raw is None:
        return None
    p = L.lib().logan_hip_moe_route_begin(0, 0, raw, k, _ptr(x), d, m)
    _write_back(descs, raw)
    if not p:
        return None
    return MoeRoutePending(p, k, d)


def moe_route_finish(pending: MoeRoutePending, out: np.ndarray) -> int:
    """logan-metal/src/lib.rs:3875-3883: 1 success, 0 decline, -1 failure."""
    out = _f32(out)
    if out.size < pending.k * pending.d:
        return 0
    raw, pending.raw = pending.raw, 0
    if not raw:
        return 0
    return int(L.lib().logan_hip_moe_route_finish(C.c_void_p(raw), _ptr(out), pending.k))


def shared_expert(descs: Sequence[MlxAffineMatmulDesc], x: np.ndarray, out: np.ndarray, d: int,
                  iinter: int) -> Optional[bool]:
    """Affine form of logan-metal/src/lib.rs:2583-2678 (shared_mxfp4):
    Ok(Some(())) -> True, Ok(None) (decline) -> None, Err(()) -> False."""
    if not hip_available() or len(descs) != 3:
        return None
    x, out = _f32(x), _f32(out)
    if x.size < d or out.size < d:
        return None
    raw, keep = _raw_descs(descs, with_y=False)
    if raw is None:
        return None
    rc = L.lib().logan_hip_shared_expert(0, 0, raw, 3, _ptr(x), _ptr(out), d, iinter)
    _write_back(descs, raw)
    if rc == 1:
        return True
    if rc == 0:
        return None
    return False


def shared_mxfp4(descs: Sequence[MetalWeightDesc], x: np.ndarray, out: np.ndarray, d: int,
                 iinter: int, model_id: int = 1, layer: int = 0) -> Optional[bool]:
    """logan-metal/src/lib.rs:2583-2678: [gate, up, down] of fmt 7 (MXFP4)
    or 21..24 (affine, fp16 sidecars); Ok(Some(())) -> True, Ok(None)
    (decline) -> None, Err(()) -> False."""
    if (not hip_available() or model_id == 0 or len(descs) != 3 or d <= 0 or iinter <= 0):
        return None
    x, out = _f32(x), _f32(out)
    if x.size < d or out.size < d:
        return None
    for dsc, (ei, eo) in zip(descs, ((d, iinter), (d, iinter), (iinter, d))):
        if dsc.i != ei or dsc.o != eo or not (dsc.fmt == 7 or 21 <= dsc.fmt <= 24):
            return None
    raw, keep = _raw_descs(descs, with_y=False)
    if raw is None:
        return None
    rc = L.lib().coli_metal_shared_mxfp4(model_id, layer, raw, 3, _ptr(x), _ptr(out), d, iinter)
    _write_back(descs, raw)
    if rc > 0:
        return True
    if rc == 0:
        return None
    return False


@dataclass
class MetalMatmulDesc:
    """logan-metal/src/lib.rs:160-168 (the llama layer's descriptors:
    fmt 5 raw bf16 weights, fmt 15 affine-8 g64 with its sidecar)."""

    tensor: Tensor
    y: np.ndarray
    weights: np.ndarray
    scales: np.ndarray
    fmt: int
    i: int
    o: int


def llama_layer(model_id: int, layer: int, descs: Sequence[MetalMatmulDesc], x: np.ndarray,
                k_out: np.ndarray, v_out: np.ndarray, input_norm: np.ndarray,
                post_norm: np.ndarray, d: int, inter: int, heads: int, kv_heads: int,
                head_dim: int, pos: int, theta: float, eps: float) -> int:
    """logan-metal/src/lib.rs:1559-1675: 1 ok, 0 declined (x untouched),
    -1 failure after submission. x [d] is updated in place; k_out / v_out
    receive the position's K (after RoPE) and V rows."""
    if (not hip_available() or model_id == 0 or len(descs) != 7 or d <= 0 or inter <= 0
            or heads <= 0 or kv_heads <= 0 or head_dim <= 0 or heads % kv_heads != 0 or pos < 0):
        return 0
    x, k_out, v_out = _f32(x), _f32(k_out), _f32(v_out)
    input_norm, post_norm = _f32(input_norm), _f32(post_norm)
    kv = kv_heads * head_dim
    if (x.size < d or k_out.size < kv or v_out.size < kv or input_norm.size < d
            or post_norm.size < d):
        return 0
    q = heads * head_dim
    expected = [(d, q), (d, kv), (d, kv), (q, d), (d, inter), (d, inter), (inter, d)]
    raw = (L.MatmulDesc * 7)()
    keep = []
    dummy = np.ones(1, np.float32)
    for k, (dsc, (ei, eo)) in enumerate(zip(descs, expected)):
        w = _bytes(dsc.weights)
        if dsc.fmt == 5:
            need_w, need_s, a = ei * eo * 2, 0, dummy.view(np.uint8)
        elif dsc.fmt == 15:
            a = _bytes(dsc.scales)
            need_w, need_s = ei * eo, 2 * eo * ((ei + 63) // 64) * 2
        else:
            return 0
        if dsc.i != ei or dsc.o != eo or w.size < need_w or a.size < need_s:
            return 0
        raw[k].tensor = dsc.tensor.handle or None
        raw[k].y = None
        raw[k].weights = _ptr(w)
        raw[k].scales = _ptr(a)
        raw[k].fmt = dsc.fmt
        raw[k].I = ei
        raw[k].O = eo
        raw[k].gs = 64 if dsc.fmt == 15 else 0
        raw[k].x = None
        raw[k].S = 1
        keep += [w, a]
    rc = L.lib().logan_hip_host_llama_layer(model_id, layer, raw, 7, _ptr(x), _ptr(k_out),
                                            _ptr(v_out), _ptr(input_norm), _ptr(post_norm), d,
                                            inter, heads, kv_heads, head_dim, pos, theta, eps)
    _write_back(descs, raw)
    return int(rc)


def llama_drop_model(model_id: int) -> None:
    """logan-metal/src/lib.rs:1677-1681."""
    if model_id and hip_available():
        L.lib().logan_hip_host_llama_drop_model(model_id)


def dense_profile_start() -> None:
    """logan-metal/src/lib.rs:772-779."""
    L.lib().logan_hip_profile_reset()
    L.lib().logan_hip_profile_set_on(1)


def dense_profile_stop():
    """logan-metal/src/lib.rs:781-789: (encode, submit, wait, kernel) ns."""
    vals = [C.c_uint64(0) for _ in range(4)]
    L.lib().logan_hip_profile_get(*[C.byref(v) for v in vals])
    L.lib().logan_hip_profile_set_on(0)
    return tuple(int(v.value) for v in vals)
