"""MUL_MAT routing over the C ABI (include/rocknpu_route.h), for numpy arrays.

A node is what the reference plugin's graph_compute reads of a ggml MUL_MAT
(adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:614-715 supports_op, :856-976
same-input grouping, :978-1650 dispatch): weight, activation and output types,
ne[], contiguity and the data pointers. `supported`, `plan` and `run` call the
library's routing functions; the arrays must outlive the call.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

F32, F16, Q4_K, Q5_K, Q6_K = 0, 1, 12, 13, 14
DECODE_CPU, DECODE_GGML, DECODE_W8A8 = 0, 1, 2
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}


class MulMatNode(ctypes.Structure):
    """rocknpu_mul_mat_node (include/rocknpu_route.h)."""

    _fields_ = [
        ("weight_type", ctypes.c_int32), ("activation_type", ctypes.c_int32), ("output_type", ctypes.c_int32),
        ("contiguous", ctypes.c_int32), ("weight_ne", ctypes.c_int64 * 4), ("activation_ne", ctypes.c_int64 * 4),
        ("weights", ctypes.c_void_p), ("weight_bytes", ctypes.c_size_t), ("activations", ctypes.c_void_p),
        ("output", ctypes.c_void_p), ("weight_name", ctypes.c_char_p),
    ]


class RouteStats(ctypes.Structure):
    """rocknpu_route_stats (include/rocknpu_route.h)."""

    _fields_ = [(name, ctypes.c_size_t) for name in (
        "graph_calls", "q4_k_mul_mat", "q5_k_mul_mat", "q6_k_mul_mat", "f16_mul_mat", "q8k_m1_mul_mat",
        "w8a8_m1_mul_mat", "mtile_group_calls", "qkv_triple_calls", "qkv_stash_hits", "graph_nodes")]
    _fields_ += [("graph_ns", ctypes.c_uint64)]
    _fields_ += [(name, ctypes.c_size_t) for name in (
        "m4_mul_mat", "m8_mul_mat", "m12_mul_mat", "m16_mul_mat", "m_other_mul_mat")]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def node(weight_type: int, weights: np.ndarray, k: int, n: int, activations: np.ndarray,
         output: np.ndarray, contiguous: bool = True, activation_type: int = F32,
         output_type: int = F32, name: str | None = None) -> MulMatNode:
    """A node for dst[m, n] = activations[m, k] x weights (K-quant blocks or
    f16 bits [n, k]); the pointers are the arrays' data, `name` the weight
    tensor's ggml name ("blk.<layer>.attn_q.weight", ...)."""
    m = activations.shape[0] if activations.ndim == 2 else 1
    nd = MulMatNode()
    nd.weight_type, nd.activation_type, nd.output_type = weight_type, activation_type, output_type
    nd.contiguous = 1 if contiguous else 0
    nd.weight_ne[:] = (k, n, 1, 1)
    nd.activation_ne[:] = (k, m, 1, 1)
    nd.weights = weights.ctypes.data
    nd.weight_bytes = weights.nbytes
    nd.activations = activations.ctypes.data
    nd.output = output.ctypes.data
    if name is not None:
        nd._name = name.encode()  # kept alive with the node
        nd.weight_name = nd._name
    return nd


def _array(nodes):
    arr = (MulMatNode * len(nodes))(*nodes)
    return arr, ctypes.cast(arr, ctypes.c_void_p)


def supported(nd: MulMatNode, decode: int = DECODE_CPU) -> bool:
    return bool(_lib.load().rocknpu_route_supported(ctypes.byref(nd), decode))


def plan(nodes, decode: int = DECODE_CPU) -> tuple[int, list[int]]:
    """(number of groups, lead index of each node's group or -1)."""
    arr, ptr = _array(nodes)
    group_of = (ctypes.c_int32 * max(1, len(nodes)))()
    groups = _lib.load().rocknpu_route_plan(ptr, len(nodes), decode, ctypes.cast(group_of, ctypes.c_void_p))
    return groups, list(group_of)[:len(nodes)]


def stats(ctx) -> dict:
    """The context's dispatch counters (rocknpu_route_stats_get)."""
    st = RouteStats()
    rc = _lib.load().rocknpu_route_stats_get(ctx.handle if hasattr(ctx, "handle") else ctx, ctypes.byref(st))
    if rc != 0:
        raise RuntimeError(f"rocknpu_route_stats_get returned {rc}")
    return st.as_dict()


def run(ctx, nodes, decode: int = DECODE_CPU) -> int:
    """Status of rocknpu_route_run on an open context (rocknpu_amd.capi.Context)."""
    arr, ptr = _array(nodes)
    return _lib.load().rocknpu_route_run(ctx.handle if hasattr(ctx, "handle") else ctx, ptr, len(nodes), decode)
