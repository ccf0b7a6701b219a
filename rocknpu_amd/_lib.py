"""ctypes binding of librocknpu_capi.so (include/rocknpu.h, rocknpu_ggml.h,
rocknpu_hip.h, rocknpu_sidecar.h, rocknpu_route.h).

The library is loaded from this package directory only. A missing library is
an error, never a fallback: every compute path in this package goes through
the gfx950 kernels.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librocknpu_capi.so"

_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p
_ctx = ctypes.c_void_p
_i = ctypes.c_int

# (name, restype, argtypes) for every exported symbol the headers declare.
SIGNATURES = {
    # rocknpu.h — the reference C ABI
    "rocknpu_device_count": (_sz, []),
    "rocknpu_context_create": (_ctx, []),
    "rocknpu_context_decode_cache_stats": (_i, [_ctx, _vp]),
    "rocknpu_context_destroy": (None, [_ctx]),
    "rocknpu_context_set_overlap": (_i, [_ctx, _vp, _vp]),
    "rocknpu_matmul_q_concat_f32_f32_mtile": (_i, [_ctx, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz]),
    "rocknpu_mtile_release": (_i, [_ctx, _sz, _vp]),
    "rocknpu_prewarm_quantized_m16": (_i, [_ctx, _vp, _sz, _u32, _sz, _sz]),
    "rocknpu_matmul_f16_f32_f32": (_i, [_ctx, _vp, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_w8a8_f32_f32_m1": (_i, [_ctx, _vp, _vp, _vp, _vp, _sz, _sz]),
    "rocknpu_matmul_w8a8_f32_f32_m16": (_i, [_ctx, _vp, _vp, _vp, _vp, _sz, _sz]),
    "rocknpu_matmul_w8a8_f32_f32_m1_nsplit": (_i, [_ctx, _vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_w8a8_swiglu_down_f32": (_i, [_ctx, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_w8a8_pair_f32_f32_m1": (_i, [_ctx, _vp, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _vp, _sz]),
    "rocknpu_matmul_q_pair_f32_f32_mtile": (
        _i, [_ctx, _vp, _sz, _u32, _sz, _vp, _sz, _u32, _sz, _vp, _vp, _vp, _sz, _sz]),
    "rocknpu_matmul_w8a8_triple_f32_f32_m1": (
        _i, [_ctx, _vp, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _sz]),
    "rocknpu_matmul_q_pair_f32_f32_m1": (_i, [_ctx, _vp, _sz, _u32, _sz, _vp, _sz, _u32, _sz, _vp, _vp, _vp, _sz]),
    "rocknpu_matmul_q_triple_f32_f32_m1": (
        _i, [_ctx, _vp, _sz, _u32, _sz, _vp, _sz, _u32, _sz, _vp, _sz, _u32, _sz, _vp, _vp, _vp, _vp, _sz]),
    "rocknpu_matmul_q4_k_f32_f32": (_i, [_ctx, _vp, _sz, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_q5_k_f32_f32": (_i, [_ctx, _vp, _sz, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_q6_k_f32_f32": (_i, [_ctx, _vp, _sz, _vp, _vp, _sz, _sz, _sz]),
    # rocknpu_ggml.h — decode MUL_MAT with llama.cpp CPU numerics
    "rocknpu_matmul_q_q8k_f32_f32": (_i, [_ctx, _u32, _vp, _sz, _vp, _vp, _sz, _sz, _sz]),
    "rocknpu_matmul_q_q8k_group_f32_f32": (_i, [_ctx, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz]),
    # rocknpu_route.h — MUL_MAT routing over the C ABI
    "rocknpu_route_supported": (_i, [_vp, ctypes.c_int32]),
    "rocknpu_route_plan": (_sz, [_vp, _sz, ctypes.c_int32, _vp]),
    "rocknpu_route_run": (_i, [_ctx, _vp, _sz, ctypes.c_int32]),
    "rocknpu_route_stats_get": (_i, [_ctx, _vp]),
    # rocknpu_sidecar.h — the W8 sidecar
    "rocknpu_w8_source_fingerprint": (ctypes.c_uint64, [_vp, _sz]),
    "rocknpu_w8_sidecar_read": (_i, [ctypes.c_char_p, ctypes.c_char_p, _vp, _sz, _sz, _sz, _vp, _vp]),
    "rocknpu_w8_sidecar_write": (_i, [ctypes.c_char_p, ctypes.c_char_p, _vp, _sz, _sz, _sz, _vp, _vp]),
    "rocknpu_w8_sidecar_get": (_i, [_ctx, ctypes.c_char_p, ctypes.c_char_p, _u32, _vp, _sz, _sz, _sz, _vp, _vp,
                                    _i, _vp]),
    # rocknpu_hip.h — device-pointer launch layer
    "rocknpu_hip_repack_w8": (_i, [_u32, _vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp]),
    "rocknpu_hip_quantize_a8": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp]),
    "rocknpu_hip_gemm_w8a8": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _vp]),
    "rocknpu_hip_gemm_route": (_i, [_sz, _sz, _sz, _i, _vp, _vp, _vp]),
    "rocknpu_hip_gemm_column_split": (_i, [_sz, _sz, _sz, _i, _vp]),
    "rocknpu_hip_gemm_w8a8_ws": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _sz, _vp]),
    "rocknpu_hip_gemm_workspace": (_i, [_sz, _sz, _sz, _i, _vp, _vp]),
    "rocknpu_hip_gemm_workspace_check": (_i, [_vp, _vp]),
    "rocknpu_hip_gemm_w8a8_tile": (_i, [_i, _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _sz,
                                        _vp]),
    "rocknpu_hip_gemv_shape": (_i, [ctypes.c_uint32, _sz, _sz, _vp, _sz, _i, _i, _vp, _vp, _vp]),
    "rocknpu_hip_quantize_q8_k": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
    "rocknpu_hip_gemv_q8_k": (_i, [_u32, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _vp]),
    "rocknpu_hip_gemv_q_f32": (_i, [_u32, _sz, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _vp]),
    "rocknpu_hip_matmul_w8a8_f32": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "rocknpu_hip_matmul_w8a8_f32_noalloc": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "rocknpu_hip_gemv_tiled_bytes": (_sz, [_u32, _sz, _sz]),
    "rocknpu_hip_gemv_tile_weights": (_i, [_u32, _vp, _sz, _sz, _sz, _vp, _sz, _vp]),
    "rocknpu_hip_gemv_q_f32_tiled": (_i, [_u32, _sz, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _vp, _sz, _vp]),
    "rocknpu_hip_gemv_q8_k_tiled": (_i, [_u32, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp]),
    "rocknpu_hip_gemv_tiled_workspace_bytes": (_sz, [_u32, _sz, _sz, _sz]),
    "rocknpu_hip_gemv_tiled_workspace_check": (_i, [_vp, _vp]),
    "rocknpu_hip_gemv_tiled_preferred": (_i, [_u32, _sz, _sz]),
    "rocknpu_hip_gemv_take_stall": (_i, []),
    "rocknpu_hip_gemv_test_stall": (_i, [_i]),
}


class DecodeCacheStats(ctypes.Structure):
    """rocknpu_decode_cache_stats (include/rocknpu.h)."""

    _fields_ = [
        ("hits", _sz), ("misses", _sz), ("entries", _sz), ("resident_bytes", _sz),
        ("hit_ns", ctypes.c_uint64), ("miss_ns", ctypes.c_uint64), ("tuned_shapes", _sz),
        ("worker1_calls", _sz), ("worker2_calls", _sz), ("worker3_calls", _sz), ("ksplit_calls", _sz),
    ]


OVERLAP_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p)

_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                " (no CPU fallback exists)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
