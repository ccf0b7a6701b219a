"""numpy-level mirror of the reference C ABI (include/rocknpu.h).

`Context` wraps one rocknpu_context; each method calls the C entry point of
the same name with host buffers and returns the status code the reference
would return (crates/rocknpu-capi/include/rocknpu.h:27-32), so tests read like
calls through the reference's FFI. Arguments that are numpy arrays must be
C-contiguous with the dtypes the header names.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

STATUS_OK = 0
STATUS_INVALID_ARGUMENT = -1
STATUS_DEVICE_ERROR = -2
STATUS_EXECUTION_ERROR = -3


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def _ptr_array(arrays):
    return (ctypes.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])


def device_count() -> int:
    return _lib.load().rocknpu_device_count()


class Context:
    """One rocknpu_context (not re-entrant, like the reference's)."""

    def __init__(self):
        self.lib = _lib.load()
        self.handle = self.lib.rocknpu_context_create()
        if not self.handle:
            raise RuntimeError("rocknpu_context_create returned NULL (no usable GPU)")
        self._overlap_keepalive = None

    def close(self):
        if self.handle:
            self.lib.rocknpu_context_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    # --- context ---------------------------------------------------------
    def decode_cache_stats(self) -> _lib.DecodeCacheStats:
        s = _lib.DecodeCacheStats()
        st = self.lib.rocknpu_context_decode_cache_stats(self.handle, ctypes.byref(s))
        if st != STATUS_OK:
            raise RuntimeError(f"decode_cache_stats status {st}")
        return s

    def set_overlap(self, fn=None) -> int:
        if fn is None:
            self._overlap_keepalive = None
            return self.lib.rocknpu_context_set_overlap(self.handle, None, None)
        cb = _lib.OVERLAP_FN(lambda _user: fn())
        self._overlap_keepalive = cb
        return self.lib.rocknpu_context_set_overlap(self.handle, ctypes.cast(cb, ctypes.c_void_p), None)

    # --- raw K-quant projections ------------------------------------------
    def matmul_q(self, kind: int, weights: np.ndarray, act: np.ndarray, out: np.ndarray, k: int, n: int) -> int:
        m = act.shape[0] if act.ndim == 2 else 1
        fn = {4: self.lib.rocknpu_matmul_q4_k_f32_f32, 5: self.lib.rocknpu_matmul_q5_k_f32_f32,
              6: self.lib.rocknpu_matmul_q6_k_f32_f32}[kind]
        return fn(self.handle, _p(weights), weights.nbytes, _p(act), _p(out), m, k, n)

    def matmul_q_q8k(self, kind: int, weights: np.ndarray, act: np.ndarray, out: np.ndarray, k: int, n: int) -> int:
        m = act.shape[0] if act.ndim == 2 else 1
        return self.lib.rocknpu_matmul_q_q8k_f32_f32(self.handle, kind, _p(weights), weights.nbytes, _p(act),
                                                     _p(out), m, k, n)

    def matmul_q_q8k_group(self, weights, kinds, ns, act: np.ndarray, outs, k: int) -> int:
        """rocknpu_matmul_q_q8k_group_f32_f32 (include/rocknpu_ggml.h)."""
        count = len(weights)
        w_arr = _ptr_array(weights)
        b_arr = (ctypes.c_size_t * count)(*[w.nbytes for w in weights])
        k_arr = (ctypes.c_uint32 * count)(*kinds)
        n_arr = (ctypes.c_size_t * count)(*ns)
        o_arr = _ptr_array(outs)
        m = act.shape[0] if act.ndim == 2 else 1
        return self.lib.rocknpu_matmul_q_q8k_group_f32_f32(self.handle, count, w_arr, b_arr, k_arr, n_arr,
                                                           _p(act), o_arr, m, k)

    def matmul_q_concat(self, weights, kinds, ns, act: np.ndarray, outs, k: int) -> int:
        count = len(weights)
        w_arr = _ptr_array(weights)
        b_arr = (ctypes.c_size_t * count)(*[w.nbytes for w in weights])
        k_arr = (ctypes.c_uint32 * count)(*kinds)
        n_arr = (ctypes.c_size_t * count)(*ns)
        o_arr = _ptr_array(outs)
        return self.lib.rocknpu_matmul_q_concat_f32_f32_mtile(self.handle, count, w_arr, b_arr, k_arr, n_arr,
                                                              _p(act), o_arr, act.shape[0], k)

    def mtile_release(self, weights) -> int:
        return self.lib.rocknpu_mtile_release(self.handle, len(weights), _ptr_array(weights))

    def prewarm_quantized_m16(self, weights: np.ndarray, kind: int, k: int, n: int) -> int:
        return self.lib.rocknpu_prewarm_quantized_m16(self.handle, _p(weights), weights.nbytes, kind, k, n)

    def matmul_q_pair_mtile(self, w1, kind1, n1, w2, kind2, n2, act, o1, o2, k) -> int:
        return self.lib.rocknpu_matmul_q_pair_f32_f32_mtile(self.handle, _p(w1), w1.nbytes, kind1, n1, _p(w2),
                                                            w2.nbytes, kind2, n2, _p(act), _p(o1), _p(o2),
                                                            act.shape[0], k)

    def matmul_q_pair_m1(self, w1, kind1, n1, w2, kind2, n2, act, o1, o2, k) -> int:
        return self.lib.rocknpu_matmul_q_pair_f32_f32_m1(self.handle, _p(w1), w1.nbytes, kind1, n1, _p(w2),
                                                         w2.nbytes, kind2, n2, _p(act), _p(o1), _p(o2), k)

    def matmul_q_triple_m1(self, w1, kind1, n1, w2, kind2, n2, w3, kind3, n3, act, o1, o2, o3, k) -> int:
        return self.lib.rocknpu_matmul_q_triple_f32_f32_m1(self.handle, _p(w1), w1.nbytes, kind1, n1, _p(w2),
                                                           w2.nbytes, kind2, n2, _p(w3), w3.nbytes, kind3, n3,
                                                           _p(act), _p(o1), _p(o2), _p(o3), k)

    # --- caller-quantised int8 projections --------------------------------
    def matmul_w8a8_m1(self, w8, scales, act, out, k, n) -> int:
        return self.lib.rocknpu_matmul_w8a8_f32_f32_m1(self.handle, _p(w8), _p(scales), _p(act), _p(out), k, n)

    def matmul_w8a8_m16(self, w8, scales, act, out, k, n) -> int:
        return self.lib.rocknpu_matmul_w8a8_f32_f32_m16(self.handle, _p(w8), _p(scales), _p(act), _p(out), k, n)

    def matmul_w8a8_m1_nsplit(self, w8, scales, act, out, k, n, chunk_n) -> int:
        return self.lib.rocknpu_matmul_w8a8_f32_f32_m1_nsplit(self.handle, _p(w8), _p(scales), _p(act), _p(out),
                                                              k, n, chunk_n)

    def matmul_w8a8_pair_m1(self, w1, s1, n1, w2, s2, n2, act, o1, o2, k) -> int:
        return self.lib.rocknpu_matmul_w8a8_pair_f32_f32_m1(self.handle, _p(w1), _p(s1), n1, _p(w2), _p(s2), n2,
                                                            _p(act), _p(o1), _p(o2), k)

    def matmul_w8a8_triple_m1(self, w1, s1, n1, w2, s2, n2, w3, s3, n3, act, o1, o2, o3, k) -> int:
        return self.lib.rocknpu_matmul_w8a8_triple_f32_f32_m1(self.handle, _p(w1), _p(s1), n1, _p(w2), _p(s2),
                                                              n2, _p(w3), _p(s3), n3, _p(act), _p(o1), _p(o2),
                                                              _p(o3), k)

    def matmul_w8a8_swiglu_down(self, gw, gs, uw, us, dw, ds, act, out, k, ffn_n, out_n) -> int:
        return self.lib.rocknpu_matmul_w8a8_swiglu_down_f32(self.handle, _p(gw), _p(gs), _p(uw), _p(us), _p(dw),
                                                            _p(ds), _p(act), _p(out), k, ffn_n, out_n)

    def matmul_f16(self, w_bits, act, out, k, n) -> int:
        return self.lib.rocknpu_matmul_f16_f32_f32(self.handle, _p(w_bits), _p(act), _p(out), act.shape[0], k, n)
