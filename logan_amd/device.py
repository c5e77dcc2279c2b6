"""Device-native (HBM-resident) entry points with torch tensors as plumbing.

torch provides device memory and streams only; every computation is a call
into liblogan_hip.so (include/logan_hip.h layer 2). A failure of the library
raises — nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib as L


class LoganHipError(RuntimeError):
    pass


def _check(rc: int, what: str) -> None:
    if rc == 1:
        return
    if rc == 0:
        raise LoganHipError(f"{what}: declined (unsupported geometry or arguments)")
    raise LoganHipError(f"{what}: device failure ({rc})")


def _stream(stream) -> Optional[int]:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None


def _where(w) -> torch.device:
    """The device holding a matrix: its tensors' device, or the `device` of a
    matrix loaded from a checkpoint (logan_amd.checkpoint)."""
    d = getattr(w, "device", None)
    if d is not None:
        return d
    t = getattr(w, "weights", None)
    return t.device if isinstance(t, torch.Tensor) else w.codes.device


def _dev(t: torch.Tensor, name: str) -> int:
    if not t.is_cuda:
        raise LoganHipError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise LoganHipError(f"{name} must be contiguous")
    return t.data_ptr()


@dataclass
class AffineMatrix:
    """One MLX-affine matrix in HBM: weights u8 [O, I*bits/8], scales/biases
    u16 (bf16 or fp16 bits) [O, I/gs]."""

    weights: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    O: int
    I: int
    bits: int
    group_size: int
    aux_fp16: bool = False

    def c(self) -> L.Affine:
        return L.Affine(_dev(self.weights, "weights"), _dev(self.scales, "scales"),
                        _dev(self.biases, "biases"), self.O, self.I, self.bits,
                        self.group_size, int(self.aux_fp16))


@dataclass
class AffineBank:
    """E stacked experts (MLX switch_mlp): weights [E, O, I*bits/8],
    scales/biases [E, O, I/gs]."""

    weights: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    E: int
    O: int
    I: int
    bits: int
    group_size: int
    aux_fp16: bool = False

    def c(self) -> L.AffineBank:
        return L.AffineBank(_dev(self.weights, "weights"), _dev(self.scales, "scales"),
                            _dev(self.biases, "biases"), self.E, self.O, self.I, self.bits,
                            self.group_size, int(self.aux_fp16))

    def expert(self, e: int) -> AffineMatrix:
        return AffineMatrix(self.weights[e], self.scales[e], self.biases[e], self.O, self.I,
                            self.bits, self.group_size, self.aux_fp16)


def affine_gemv(w: AffineMatrix, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                out_dtype: torch.dtype = torch.bfloat16, stream=None) -> torch.Tensor:
    """y[M, O] = x[M, I] . W^T, x bf16 (logan-qwen4/src/lib.rs:3729-3764)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    x2 = x.reshape(-1, w.I)
    M = x2.shape[0]
    if out is None:
        out = torch.empty((M, w.O), dtype=out_dtype, device=x.device)
    yd = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("out must be bf16 or f32")
    a = w.c()
    rc = L.lib().logan_hip_affine_gemv(C.byref(a), _dev(x2, "x"), M, w.I, _dev(out, "out"), w.O,
                                       yd, _stream(stream))
    _check(rc, "affine_gemv")
    return out


def affine_gemv_multi(ws, x: torch.Tensor, outs=None, out_dtype: torch.dtype = torch.bfloat16,
                      stream=None):
    """Matrices sharing one activation in one launch (up to 8): returns
    [x . W_i^T] (logan-metal/metal/backend_metal.mm:2290-2493)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    if not 1 <= len(ws) <= 8:
        raise LoganHipError("between 1 and 8 matrices")
    x2 = x.reshape(-1, ws[0].I)
    M = x2.shape[0]
    if outs is None:
        outs = [torch.empty((M, w.O), dtype=out_dtype, device=x.device) for w in ws]
    dts = {o.dtype for o in outs}
    if len(dts) != 1 or next(iter(dts)) not in (torch.bfloat16, torch.float32):
        raise LoganHipError("outputs must all be bf16 or all f32")
    yd = L.LOGAN_HIP_BF16 if outs[0].dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    arr = (L.Affine * len(ws))(*[w.c() for w in ws])
    ptrs = (C.c_void_p * len(ws))(*[_dev(o, "out") for o in outs])
    rc = L.lib().logan_hip_affine_gemv_multi(arr, len(ws), _dev(x2, "x"), M, ws[0].I, ptrs, yd,
                                             _stream(stream))
    _check(rc, "affine_gemv_multi")
    return outs


def affine_qmm(w: AffineMatrix, x: torch.Tensor, out: Optional[torch.Tensor] = None,
               out_dtype: torch.dtype = torch.bfloat16, stream=None) -> torch.Tensor:
    """Prefill product on MFMA with the reference QMM numerics: y[M, O] =
    x[M, I] . bf16(W)^T (logan-metal/metal/backend_metal.mm:1480-1560)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    x2 = x.reshape(-1, w.I)
    M = x2.shape[0]
    if out is None:
        out = torch.empty((M, w.O), dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("out must be bf16 or f32")
    yd = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    a = w.c()
    rc = L.lib().logan_hip_affine_qmm(C.byref(a), _dev(x2, "x"), M, w.I, _dev(out, "out"), w.O,
                                      yd, _stream(stream))
    _check(rc, "affine_qmm")
    return out


def affine_gemv_swiglu(gate: AffineMatrix, up: AffineMatrix, x: torch.Tensor,
                       out: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
                       stream=None) -> torch.Tensor:
    """h[M, O] = silu(x . gate^T) * (x . up^T) in one product
    (logan-qwen4/src/lib.rs:8803-8812)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    x2 = x.reshape(-1, gate.I)
    M = x2.shape[0]
    if out is None:
        out = torch.empty((M, gate.O), dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("out must be bf16 or f32")
    hd = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    g, u = gate.c(), up.c()
    rc = L.lib().logan_hip_affine_gemv_swiglu(C.byref(g), C.byref(u), _dev(x2, "x"), M, gate.I,
                                              _dev(out, "out"), gate.O, hd, _stream(stream))
    _check(rc, "affine_gemv_swiglu")
    return out


def affine_qmm_multi(ws, x: torch.Tensor, outs=None, out_dtype: torch.dtype = torch.bfloat16,
                     stream=None):
    """Prefill products of up to 8 matrices sharing x in one grid: returns
    [x . bf16(W_i)^T] (the QMM numerics of affine_qmm)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    if not 1 <= len(ws) <= 8:
        raise LoganHipError("between 1 and 8 matrices")
    x2 = x.reshape(-1, ws[0].I)
    M = x2.shape[0]
    if outs is None:
        outs = [torch.empty((M, w.O), dtype=out_dtype, device=x.device) for w in ws]
    dts = {o.dtype for o in outs}
    if len(dts) != 1 or next(iter(dts)) not in (torch.bfloat16, torch.float32):
        raise LoganHipError("outputs must all be bf16 or all f32")
    yd = L.LOGAN_HIP_BF16 if outs[0].dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    arr = (L.Affine * len(ws))(*[w.c() for w in ws])
    ptrs = (C.c_void_p * len(ws))(*[_dev(o, "out") for o in outs])
    rc = L.lib().logan_hip_affine_qmm_multi(arr, len(ws), _dev(x2, "x"), M, ws[0].I, ptrs, yd,
                                            _stream(stream))
    _check(rc, "affine_qmm_multi")
    return outs


def silu_mul(g: torch.Tensor, u: torch.Tensor, stream=None) -> torch.Tensor:
    """In place g = silu(g) * u (f32 or bf16 device tensors of equal size;
    logan-metal/metal/backend_metal.mm:2187-2203). Returns g."""
    if g.dtype != u.dtype or g.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("g and u must both be bf16 or both f32")
    if g.numel() != u.numel():
        raise LoganHipError("g and u differ in size")
    dt = L.LOGAN_HIP_BF16 if g.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    rc = L.lib().logan_hip_silu_mul(_dev(g, "g"), _dev(u, "u"), g.numel(), dt, _stream(stream))
    _check(rc, "silu_mul")
    return g


def affine_gemv_f32(w: AffineMatrix, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                    stream=None) -> torch.Tensor:
    """f32 activations, exact per-element dequantisation, f32 output."""
    if x.dtype != torch.float32:
        raise LoganHipError("x must be f32")
    x2 = x.reshape(-1, w.I)
    M = x2.shape[0]
    if out is None:
        out = torch.empty((M, w.O), dtype=torch.float32, device=x.device)
    a = w.c()
    rc = L.lib().logan_hip_affine_gemv_f32(C.byref(a), _dev(x2, "x"), M, w.I, _dev(out, "out"),
                                           w.O, _stream(stream))
    _check(rc, "affine_gemv_f32")
    return out


def affine_dequant(w: AffineMatrix, row0: int = 0, nrows: Optional[int] = None,
                   stream=None) -> torch.Tensor:
    """code*scale+bias as f32 for rows [row0, row0+nrows)."""
    n = w.O - row0 if nrows is None else nrows
    out = torch.empty((n, w.I), dtype=torch.float32, device=_where(w))
    a = w.c()
    rc = L.lib().logan_hip_affine_dequant(C.byref(a), row0, n, _dev(out, "out"), _stream(stream))
    _check(rc, "affine_dequant")
    return out


@dataclass
class Mxfp4Matrix:
    """One MXFP4 matrix in HBM (logan-metal fmt 7; planes 2 / 3 = fmt 9 /
    10): codes u8 [planes, O, I/2], E8M0 scale bytes u8 [planes, O, I/32]."""

    codes: torch.Tensor
    scales: torch.Tensor
    O: int
    I: int
    planes: int = 1

    def c(self) -> L.Mxfp4:
        return L.Mxfp4(_dev(self.codes, "codes"), _dev(self.scales, "scales"), self.O, self.I,
                       self.planes)


def mxfp4_gemv(ws, xs, outs=None, out_dtype: torch.dtype = torch.float32, stream=None):
    """[W_i . x_i] for up to 16 MXFP4 matrices, each with its own activation
    (one row, f32 or bf16), in one launch (backend_metal.mm:438-490)."""
    if not 1 <= len(ws) <= 16 or len(xs) != len(ws):
        raise LoganHipError("between 1 and 16 matrices, one activation each")
    dts = {x.dtype for x in xs}
    if len(dts) != 1 or next(iter(dts)) not in (torch.bfloat16, torch.float32):
        raise LoganHipError("activations must all be bf16 or all f32")
    for w, x in zip(ws, xs):
        if x.numel() != w.I:
            raise LoganHipError("activation length must equal I")
    if outs is None:
        outs = [torch.empty(w.O, dtype=out_dtype, device=xs[0].device) for w in ws]
    ods = {o.dtype for o in outs}
    if len(ods) != 1 or next(iter(ods)) not in (torch.bfloat16, torch.float32):
        raise LoganHipError("outputs must all be bf16 or all f32")
    xd = L.LOGAN_HIP_BF16 if xs[0].dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    yd = L.LOGAN_HIP_BF16 if outs[0].dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    arr = (L.Mxfp4 * len(ws))(*[w.c() for w in ws])
    xp = (C.c_void_p * len(ws))(*[_dev(x, "x") for x in xs])
    yp = (C.c_void_p * len(ws))(*[_dev(o, "out") for o in outs])
    rc = L.lib().logan_hip_mxfp4_gemv(arr, len(ws), xp, xd, yp, yd, _stream(stream))
    _check(rc, "mxfp4_gemv")
    return outs


def mxfp4_dequant(w: Mxfp4Matrix, row0: int = 0, nrows: Optional[int] = None,
                  stream=None) -> torch.Tensor:
    """E2M1(code) * 2^(scale - 127) of plane 0 as f32, rows [row0, row0+nrows)."""
    n = w.O - row0 if nrows is None else nrows
    out = torch.empty((n, w.I), dtype=torch.float32, device=_where(w))
    a = w.c()
    rc = L.lib().logan_hip_mxfp4_dequant(C.byref(a), row0, n, _dev(out, "out"), _stream(stream))
    _check(rc, "mxfp4_dequant")
    return out


@dataclass
class DenseMatrix:
    """One matrix of the dense decode layer in HBM: fmt 5 weights bf16
    [O, I]; fmt 15 affine-8 codes u8 [O, I] with bf16 scales / biases
    [O, I/64]."""

    weights: torch.Tensor
    O: int
    I: int
    fmt: int
    scales: Optional[torch.Tensor] = None
    biases: Optional[torch.Tensor] = None

    def c(self) -> L.Dense:
        sc = _dev(self.scales, "scales") if self.scales is not None else None
        bi = _dev(self.biases, "biases") if self.biases is not None else None
        return L.Dense(_dev(self.weights, "weights"), sc, bi, self.O, self.I, self.fmt)


@dataclass
class LlamaLayer:
    """A dense Llama layer in HBM with its f32 K/V cache
    [cache_tokens, kv_heads * head_dim] (logan-metal/metal/backend_metal.mm
    :2495-2791)."""

    mats: list  # q, k, v, o, gate, up, down (DenseMatrix)
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    D: int
    inter: int
    heads: int
    kv_heads: int
    head_dim: int
    theta: float
    eps: float

    def c(self) -> L.LlamaLayer:
        m = [x.c() for x in self.mats]
        return L.LlamaLayer(*m, _dev(self.in_norm, "in_norm"), _dev(self.post_norm, "post_norm"),
                            _dev(self.k_cache, "k_cache"), _dev(self.v_cache, "v_cache"),
                            self.k_cache.shape[0], self.D, self.inter, self.heads, self.kv_heads,
                            self.head_dim, self.theta, self.eps)


def llama_workspace_bytes(layer: LlamaLayer, pos: int) -> int:
    c = layer.c()
    return int(L.lib().logan_hip_llama_workspace_bytes(C.byref(c), pos))


def llama_layer(layer: LlamaLayer, x: torch.Tensor, pos: int, workspace=None, stream=None):
    """x [D] f32 in place: one decode layer at position pos; K/V rows land in
    the layer's caches at row pos."""
    if x.dtype != torch.float32 or x.numel() != layer.D:
        raise LoganHipError("x must be f32 [D]")
    c = layer.c()
    need = int(L.lib().logan_hip_llama_workspace_bytes(C.byref(c), pos))
    if need == 0:
        raise LoganHipError("llama_layer: unsupported layer")
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    rc = L.lib().logan_hip_llama_layer(C.byref(c), _dev(x, "x"), pos, _dev(workspace, "workspace"),
                                       workspace.numel(), _stream(stream))
    _check(rc, "llama_layer")
    return x


def route_topk(logits: torch.Tensor, k: int, stream=None):
    """Per row: softmax top-k, lower-index ties; returns (idx int32 [B,k],
    weights f32 [B,k])."""
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("logits must be bf16 or f32")
    B, E = logits.shape
    idx = torch.empty((B, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((B, k), dtype=torch.float32, device=logits.device)
    dt = L.LOGAN_HIP_BF16 if logits.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    rc = L.lib().logan_hip_route_topk(_dev(logits, "logits"), dt, B, E, k, _dev(idx, "idx"),
                                      _dev(w, "w"), _stream(stream))
    _check(rc, "route_topk")
    return idx, w


@dataclass
class MoeLayer:
    """Routed experts + optional shared expert of one MoE block."""

    gate: AffineBank
    up: AffineBank
    down: AffineBank
    top_k: int
    shared_gate: Optional[AffineBank] = None
    shared_up: Optional[AffineBank] = None
    shared_down: Optional[AffineBank] = None
    shared_gate_vec: Optional[torch.Tensor] = None  # bf16 [D]

    def c(self) -> L.MoeBlock:
        blk = L.MoeBlock()
        blk.gate, blk.up, blk.down = self.gate.c(), self.up.c(), self.down.c()
        if self.shared_gate is not None:
            blk.shared_gate = self.shared_gate.c()
            blk.shared_up = self.shared_up.c()
            blk.shared_down = self.shared_down.c()
        blk.shared_gate_vec = (_dev(self.shared_gate_vec, "shared_gate_vec")
                               if self.shared_gate_vec is not None else None)
        blk.top_k = self.top_k
        return blk

    def workspace_bytes(self, B: int) -> int:
        blk = self.c()
        return int(L.lib().logan_hip_moe_workspace_bytes(C.byref(blk), B))


def moe_block(layer: MoeLayer, x: torch.Tensor, logits: torch.Tensor,
              out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
              return_routing: bool = False, out_dtype: torch.dtype = torch.bfloat16,
              stream=None):
    """out[B, D] = routed MoE + shared expert (logan-qwen/src/lib.rs:535-593),
    bf16 (RNE of the f32 result) or f32."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("logits must be bf16 or f32")
    B, D = x.shape
    if out is None:
        out = torch.empty((B, D), dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("out must be bf16 or f32")
    od = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    idx = w = None
    if return_routing:
        idx = torch.empty((B, layer.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((B, layer.top_k), dtype=torch.float32, device=x.device)
    blk = layer.c()
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = _dev(workspace, "workspace"), workspace.numel() * workspace.element_size()
    dt = L.LOGAN_HIP_BF16 if logits.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    rc = L.lib().logan_hip_moe_block(C.byref(blk), _dev(x, "x"), _dev(logits, "logits"), dt, B,
                                     _dev(out, "out"), od,
                                     idx.data_ptr() if idx is not None else None,
                                     w.data_ptr() if w is not None else None, ws_ptr, ws_bytes,
                                     _stream(stream))
    _check(rc, "moe_block")
    if return_routing:
        return out, idx, w
    return out


def moe_block_cached(layer: MoeLayer, cache, experts, blocks, x: torch.Tensor,
                     logits: torch.Tensor, out: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None, return_routing: bool = False,
                     out_dtype: torch.dtype = torch.bfloat16, stream=None):
    """moe_block for one token whose routed experts sit in an ExpertCache
    (logan_amd.checkpoint): experts / blocks are the route and the blocks
    ExpertCache.fetch returned; layer supplies top_k, the shared expert and
    the routed geometry (logan_hip_moe_block_cached)."""
    if x.dtype != torch.bfloat16 or x.numel() != x.shape[-1]:
        raise LoganHipError("x must be one bf16 token")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("logits must be bf16 or f32")
    D = x.shape[-1]
    if out is None:
        out = torch.empty((1, D), dtype=out_dtype, device=x.device)
    od = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    e = np.ascontiguousarray(experts, dtype=np.int32)
    b = np.ascontiguousarray(blocks, dtype=np.int32)
    if len(e) != len(b):
        raise LoganHipError("experts and blocks differ in length")
    idx = w = None
    if return_routing:
        idx = torch.empty((1, layer.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((1, layer.top_k), dtype=torch.float32, device=x.device)
    blk = layer.c()
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = _dev(workspace, "workspace"), workspace.numel() * workspace.element_size()
    dt = L.LOGAN_HIP_BF16 if logits.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    rc = L.lib().logan_hip_moe_block_cached(C.byref(blk), cache.handle, e.ctypes.data, b.ctypes.data,
                                            len(e), _dev(x, "x"), _dev(logits, "logits"), dt,
                                            _dev(out, "out"), od,
                                            idx.data_ptr() if idx is not None else None,
                                            w.data_ptr() if w is not None else None, ws_ptr,
                                            ws_bytes, _stream(stream))
    _check(rc, "moe_block_cached")
    if return_routing:
        return out, idx, w
    return out


def moe_block_routed(layer: MoeLayer, router: AffineMatrix, x: torch.Tensor,
                     out: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None, return_routing: bool = False,
                     out_dtype: torch.dtype = torch.bfloat16, stream=None):
    """moe_block with the router product on device (logan_hip_moe_block_routed):
    logits = x . router^T in f32 (returned), then the block on them."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    B, D = x.shape
    if out is None:
        out = torch.empty((B, D), dtype=out_dtype, device=x.device)
    if logits is None:
        logits = torch.empty((B, router.O), dtype=torch.float32, device=x.device)
    od = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    idx = w = None
    if return_routing:
        idx = torch.empty((B, layer.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((B, layer.top_k), dtype=torch.float32, device=x.device)
    blk = layer.c()
    rt = router.c()
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = _dev(workspace, "workspace"), workspace.numel() * workspace.element_size()
    rc = L.lib().logan_hip_moe_block_routed(C.byref(blk), C.byref(rt), _dev(x, "x"), B,
                                            _dev(logits, "logits"), _dev(out, "out"), od,
                                            idx.data_ptr() if idx is not None else None,
                                            w.data_ptr() if w is not None else None, ws_ptr,
                                            ws_bytes, _stream(stream))
    _check(rc, "moe_block_routed")
    if return_routing:
        return out, logits, idx, w
    return out, logits


def moe_block_static(layer: MoeLayer, x: torch.Tensor, logits: torch.Tensor,
                     out: Optional[torch.Tensor] = None, return_routing: bool = False,
                     out_dtype: torch.dtype = torch.bfloat16, stream=None):
    """moe_block on the library's static device scratch (no workspace, no
    allocation inside the call; logan_hip_moe_block_static)."""
    if x.dtype != torch.bfloat16:
        raise LoganHipError("x must be bf16")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("logits must be bf16 or f32")
    B, D = x.shape
    if out is None:
        out = torch.empty((B, D), dtype=out_dtype, device=x.device)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise LoganHipError("out must be bf16 or f32")
    od = L.LOGAN_HIP_BF16 if out.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    idx = w = None
    if return_routing:
        idx = torch.empty((B, layer.top_k), dtype=torch.int32, device=x.device)
        w = torch.empty((B, layer.top_k), dtype=torch.float32, device=x.device)
    blk = layer.c()
    dt = L.LOGAN_HIP_BF16 if logits.dtype == torch.bfloat16 else L.LOGAN_HIP_F32
    rc = L.lib().logan_hip_moe_block_static(C.byref(blk), _dev(x, "x"), _dev(logits, "logits"), dt,
                                            B, _dev(out, "out"), od,
                                            idx.data_ptr() if idx is not None else None,
                                            w.data_ptr() if w is not None else None,
                                            _stream(stream))
    _check(rc, "moe_block_static")
    if return_routing:
        return out, idx, w
    return out
