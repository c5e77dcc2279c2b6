"""ctypes binding of liblogan_hip.so (the C ABI in include/logan_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "liblogan_hip.so"

LOGAN_HIP_F32 = 0
LOGAN_HIP_BF16 = 1
LOGAN_HIP_WT_AFFINE = 1
LOGAN_HIP_WT_MXFP4 = 2


class MatmulDesc(C.Structure):
    """LoganHipMatmulDesc == ColiMetalMatmulDesc (backend_metal.h:68-88)."""

    _fields_ = [
        ("tensor", C.c_void_p),
        ("y", C.c_void_p),
        ("weights", C.c_void_p),
        ("scales", C.c_void_p),
        ("fmt", C.c_int),
        ("I", C.c_int),
        ("O", C.c_int),
        ("gs", C.c_int),
        ("x", C.c_void_p),
        ("S", C.c_int),
    ]


class Affine(C.Structure):
    _fields_ = [
        ("weights", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("O", C.c_int),
        ("I", C.c_int),
        ("bits", C.c_int),
        ("group_size", C.c_int),
        ("aux_fp16", C.c_int),
    ]


class Mxfp4(C.Structure):
    _fields_ = [
        ("codes", C.c_void_p),
        ("scales", C.c_void_p),
        ("O", C.c_int),
        ("I", C.c_int),
        ("planes", C.c_int),
    ]


class Dense(C.Structure):
    _fields_ = [
        ("weights", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("O", C.c_int),
        ("I", C.c_int),
        ("fmt", C.c_int),
    ]


class LlamaLayer(C.Structure):
    _fields_ = [(n, Dense) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("in_norm", C.c_void_p),
        ("post_norm", C.c_void_p),
        ("k_cache", C.c_void_p),
        ("v_cache", C.c_void_p),
        ("cache_tokens", C.c_int),
        ("D", C.c_int),
        ("inter", C.c_int),
        ("heads", C.c_int),
        ("kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("theta", C.c_float),
        ("eps", C.c_float),
    ]


class AffineBank(C.Structure):
    _fields_ = [
        ("weights", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("E", C.c_int),
        ("O", C.c_int),
        ("I", C.c_int),
        ("bits", C.c_int),
        ("group_size", C.c_int),
        ("aux_fp16", C.c_int),
    ]


class MoeBlock(C.Structure):
    _fields_ = [
        ("gate", AffineBank),
        ("up", AffineBank),
        ("down", AffineBank),
        ("shared_gate", AffineBank),
        ("shared_up", AffineBank),
        ("shared_down", AffineBank),
        ("shared_gate_vec", C.c_void_p),
        ("top_k", C.c_int),
    ]


class QuantWt(C.Structure):
    _fields_ = [
        ("kind", C.c_int),
        ("E", C.c_int),
        ("O", C.c_int),
        ("I", C.c_int),
        ("bits", C.c_int),
        ("group_size", C.c_int),
        ("aux_fp16", C.c_int),
        ("weights", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("weight_bytes", C.c_uint64),
        ("scale_bytes", C.c_uint64),
        ("bias_bytes", C.c_uint64),
        ("owner", C.c_void_p),
    ]


class ExpertCacheStats(C.Structure):
    _fields_ = [
        ("hits", C.c_uint64),
        ("misses", C.c_uint64),
        ("evictions", C.c_uint64),
        ("streamed", C.c_uint64),
        ("bytes_loaded", C.c_uint64),
        ("generation", C.c_uint64),
        ("block_bytes", C.c_uint64),
        ("device_bytes", C.c_uint64),
        ("layers", C.c_int),
        ("blocks_per_layer", C.c_int),
        ("topk", C.c_int),
    ]


_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_U64 = C.c_uint64

# name -> (restype, argtypes)
SIGNATURES = {
    "logan_hip_init": (_I, []),
    "logan_hip_available": (_I, []),
    "logan_hip_shutdown": (None, []),
    "logan_hip_stats": (None, [C.POINTER(_SZ), C.POINTER(_SZ)]),
    "logan_hip_mem_info": (_I, [C.POINTER(_SZ), C.POINTER(_SZ)]),
    "logan_hip_profile_set_on": (None, [_I]),
    "logan_hip_profile_reset": (None, []),
    "logan_hip_profile_get": (None, [C.POINTER(_U64)] * 4),
    "logan_hip_matmul": (_I, [C.POINTER(_P), _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "logan_hip_matmul_multi": (_I, [_P, _I, C.POINTER(MatmulDesc), _I]),
    "logan_hip_moe_route_begin": (_P, [_U64, _I, C.POINTER(MatmulDesc), _I, _P, _I, _I]),
    "logan_hip_moe_route_finish": (_I, [_P, _P, _I]),
    "logan_hip_moe_route_discard": (None, [_P]),
    "logan_hip_moe_route_drop_model": (None, [_U64]),
    "logan_hip_shared_expert": (_I, [_U64, _I, C.POINTER(MatmulDesc), _I, _P, _P, _I, _I]),
    # logan-metal's own name for the shared-expert entry (include/logan_metal_ffi.h)
    "coli_metal_shared_mxfp4": (_I, [_U64, _I, C.POINTER(MatmulDesc), _I, _P, _P, _I, _I]),
    "logan_hip_shared_expert_drop_model": (None, [_U64]),
    "logan_hip_host_rmsnorm": (_I, [_P, _P, _I, _I, C.c_float]),
    "logan_hip_host_add": (_I, [_P, _P, _I]),
    "logan_hip_host_silu_mul": (_I, [_P, _P, _I]),
    "logan_hip_tensor_free": (None, [_P]),
    "logan_hip_tensor_bytes": (_SZ, [_P]),
    "logan_hip_affine_gemv": (_I, [C.POINTER(Affine), _P, _I, _I, _P, _I, _I, _P]),
    "logan_hip_affine_gemv_f32": (_I, [C.POINTER(Affine), _P, _I, _I, _P, _I, _P]),
    "logan_hip_affine_gemv_multi": (_I, [C.POINTER(Affine), _I, _P, _I, _I, C.POINTER(_P), _I, _P]),
    "logan_hip_affine_gemv_swiglu": (_I, [C.POINTER(Affine), C.POINTER(Affine), _P, _I, _I, _P, _I,
                                          _I, _P]),
    "logan_hip_affine_qmm": (_I, [C.POINTER(Affine), _P, _I, _I, _P, _I, _I, _P]),
    "logan_hip_affine_qmm_multi": (_I, [C.POINTER(Affine), _I, _P, _I, _I, C.POINTER(_P), _I, _P]),
    "logan_hip_silu_mul": (_I, [_P, _P, C.c_longlong, _I, _P]),
    "logan_hip_affine_dequant": (_I, [C.POINTER(Affine), _I, _I, _P, _P]),
    "logan_hip_mxfp4_gemv": (_I, [C.POINTER(Mxfp4), _I, C.POINTER(C.c_void_p), _I,
                                  C.POINTER(C.c_void_p), _I, _P]),
    "logan_hip_mxfp4_dequant": (_I, [C.POINTER(Mxfp4), _I, _I, _P, _P]),
    "logan_hip_llama_workspace_bytes": (_SZ, [C.POINTER(LlamaLayer), _I]),
    "logan_hip_llama_layer": (_I, [C.POINTER(LlamaLayer), _P, _I, _P, _SZ, _P]),
    "logan_hip_host_llama_layer": (_I, [_U64, _I, C.POINTER(MatmulDesc), _I, _P, _P, _P, _P, _P,
                                        _I, _I, _I, _I, _I, _I, C.c_float, C.c_float]),
    "logan_hip_host_llama_drop_model": (None, [_U64]),
    "logan_hip_route_topk": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "logan_hip_moe_workspace_bytes": (_SZ, [C.POINTER(MoeBlock), _I]),
    "logan_hip_moe_block": (_I, [C.POINTER(MoeBlock), _P, _P, _I, _I, _P, _I, _P, _P, _P, _SZ, _P]),
    "logan_hip_moe_block_routed": (_I, [C.POINTER(MoeBlock), C.POINTER(Affine), _P, _I, _P, _P, _I, _P,
                                        _P, _P, _SZ, _P]),
    "logan_hip_moe_block_static": (_I, [C.POINTER(MoeBlock), _P, _P, _I, _I, _P, _I, _P, _P, _P]),
    "logan_hip_set_moe_fused": (None, [_I]),
    "logan_hip_set_moe_mfma_min_batch": (None, [_I]),
    "logan_hip_moe_sync_errors": (C.c_uint32, []),
    "logan_hip_version": (C.c_char_p, []),
    "logan_hip_last_error": (C.c_char_p, []),
    "logan_hip_st_open": (_P, [C.c_char_p]),
    "logan_hip_st_open_dir": (_P, [C.c_char_p]),
    "logan_hip_st_close": (None, [_P]),
    "logan_hip_st_shard_count": (_I, [_P]),
    "logan_hip_st_tensor": (_I, [_P, C.c_char_p, C.c_char_p, _SZ, C.POINTER(_U64), _I,
                                 C.POINTER(_I), C.POINTER(_U64)]),
    "logan_hip_st_dtype_count": (_I, [_P, C.c_char_p]),
    "logan_hip_st_read": (_I, [_P, C.c_char_p, _U64, _U64, _P]),
    "logan_hip_load_mlx_quantized": (_I, [_P, C.c_char_p, _I, _I, C.POINTER(QuantWt)]),
    "logan_hip_load_mlx_quantized_experts": (_I, [_P, C.c_char_p, _I, _I, _I, _I, _I,
                                                  C.POINTER(QuantWt)]),
    "logan_hip_plan_mlx_quantized": (_I, [_P, C.c_char_p, _I, _I, C.POINTER(QuantWt)]),
    "logan_hip_plan_mlx_quantized_experts": (_I, [_P, C.c_char_p, _I, _I, _I, _I, _I,
                                                  C.POINTER(QuantWt)]),
    "logan_hip_quant_free": (None, [C.POINTER(QuantWt)]),
    "logan_hip_expert_cache_create": (_P, [_P, _I, _I, _I, _I, _I, _I]),
    "logan_hip_expert_cache_destroy": (None, [_P]),
    "logan_hip_expert_cache_fetch": (_I, [_P, _I, _P, _I, _P, _P]),
    "logan_hip_expert_cache_stats": (None, [_P, C.POINTER(ExpertCacheStats)]),
    "logan_hip_expert_cache_tags": (_I, [_P, _I, _P]),
    "logan_hip_moe_block_cached": (_I, [C.POINTER(MoeBlock), _P, _P, _P, _I, _P, _P, _I, _P, _I, _P,
                                        _P, _P, _SZ, _P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it was not built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("LOGAN_HIP_LIB", LIB_PATH))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python logan_amd/build.py` "
                "(logan-hip has no CPU fallback)"
            )
        handle = C.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib
