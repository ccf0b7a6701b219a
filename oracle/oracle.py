"""ctypes wrapper of the C oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; nothing in the product imports it. The C functions and the
reference lines they restate are listed in oracle.h.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

QK = 256
BLOCK_BYTES = {4: 144, 5: 176, 6: 210}
Q8K_BYTES = 292

_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_sz = ctypes.c_size_t


class OracleError(RuntimeError):
    """The oracle returned a non-zero status (the reference's -1)."""


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def use_native_build(out_dir: str) -> Path:
    """Compile oracle.c for this host's CPU (-march=native, the same
    floating-point flags) into out_dir and make it the library the functions
    below call. For timing the CPU baseline on the machine it runs on."""
    out = Path(out_dir) / "liboracle_native.so"
    subprocess.run(["gcc", "-O3", "-march=native", "-std=gnu11", "-fPIC", "-fopenmp", "-ffp-contract=off",
                    "-fno-fast-math", "-shared", "-o", str(out), str(HERE / "oracle.c"), "-lm"], check=True)
    global _lib
    _lib = _configure(ctypes.CDLL(str(out)))
    return out


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _configure(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def _configure(L: ctypes.CDLL) -> ctypes.CDLL:
    L.or_fp16_to_f32.argtypes = [ctypes.c_uint16]
    L.or_fp16_to_f32.restype = ctypes.c_float
    L.or_dequant_rows.argtypes = [ctypes.c_uint32, _u8p, _sz, _sz, _f32p]
    L.or_quantize_symmetric_row.argtypes = [_f32p, _sz, _i8p, _f32p]
    L.or_quantize_symmetric_row_neon.argtypes = [_f32p, _sz, _i8p, _f32p]
    L.or_rescale_neon.argtypes = [_i32p, _f32p, _f32p, _sz, _sz, _f32p]
    L.or_rescale_neon.restype = None
    L.or_repack_w8.argtypes = [ctypes.c_uint32, _u8p, _sz, _sz, _sz, _i8p, _f32p]
    L.or_quantize_a8.argtypes = [_f32p, _sz, _sz, _sz, _i8p, _f32p]
    L.or_gemm_i32.argtypes = [_i8p, _i8p, _sz, _sz, _sz, _i32p, ctypes.c_int]
    L.or_gemm_i32.restype = None
    L.or_rescale.argtypes = [_i32p, _f32p, _f32p, _sz, _sz, _f32p]
    L.or_rescale.restype = None
    L.or_matmul_q_w8a8.argtypes = [ctypes.c_uint32, _u8p, _sz, _f32p, _sz, _sz, _sz, _f32p, ctypes.c_int]
    L.or_fnv1a64.argtypes = [ctypes.c_uint64, _u8p, _sz]
    L.or_fnv1a64.restype = ctypes.c_uint64
    L.or_source_fingerprint.argtypes = [_u8p, _sz]
    L.or_source_fingerprint.restype = ctypes.c_uint64
    L.or_hilo_stack.argtypes = [_f32p, _sz, _sz, _f32p]
    L.or_hilo_sum.argtypes = [_f32p, _f32p, _sz]
    L.or_hilo_sum.restype = None
    L.or_quantize_row_q8_k.argtypes = [_f32p, _sz, _u8p]
    L.or_quantize_row_q8_k.restype = None
    L.or_vec_dot_q4_k_q8_k.argtypes = [_sz, _u8p, _u8p]
    L.or_vec_dot_q4_k_q8_k.restype = ctypes.c_float
    L.or_vec_dot_q6_k_q8_k.argtypes = [_sz, _u8p, _u8p]
    L.or_vec_dot_q6_k_q8_k.restype = ctypes.c_float
    L.or_gemv_q8_k.argtypes = [ctypes.c_uint32, _u8p, _sz, _sz, _u8p, _sz, _f32p, ctypes.c_int]
    L.or_gemv_block_sums.argtypes = [ctypes.c_uint32, _u8p, _sz, _sz, _u8p, _i32p, _i32p, _f64p]
    return L


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(t)


def fp16_to_f32(bits: int) -> float:
    return lib().or_fp16_to_f32(bits)


def dequant_rows(kind: int, blocks: np.ndarray, k: int, n: int) -> np.ndarray:
    out = np.empty((n, k), np.float32)
    if lib().or_dequant_rows(kind, _p(blocks, _u8p), k, n, _p(out, _f32p)) != 0:
        raise OracleError("dequant_rows")
    return out


def quantize_symmetric_row(x: np.ndarray, neon: bool = False):
    """The reference's symmetric row quantisation; neon=True gives its aarch64
    NEON form (multiply by the reciprocal scale in chunks of 8)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.size, np.int8)
    s = ctypes.c_float()
    fn = lib().or_quantize_symmetric_row_neon if neon else lib().or_quantize_symmetric_row
    if fn(_p(x, _f32p), x.size, _p(q, _i8p), ctypes.byref(s)) != 0:
        raise OracleError("non-finite row")
    return q, np.float32(s.value)


def repack_w8(kind: int, blocks: np.ndarray, k: int, n: int, threads: int = 1):
    """W8 [n, k] + scales [n]. threads > 1 repacks row ranges concurrently
    (rows are independent; the C call releases the GIL)."""
    w8 = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    flat = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    row_bytes = (k // QK) * BLOCK_BYTES.get(kind, 0)

    def one(r0, r1):
        part = flat[r0 * row_bytes:r1 * row_bytes] if row_bytes else flat
        return lib().or_repack_w8(kind, _p(part, _u8p), part.nbytes, k, r1 - r0, _p(w8[r0:r1], _i8p),
                                  _p(sc[r0:r1], _f32p))

    if threads <= 1 or n < 2 * threads or row_bytes == 0 or flat.nbytes != n * row_bytes:
        rcs = [one(0, n)]
    else:
        from concurrent.futures import ThreadPoolExecutor
        step = (n + threads - 1) // threads
        with ThreadPoolExecutor(threads) as pool:
            rcs = list(pool.map(lambda r0: one(r0, min(n, r0 + step)), range(0, n, step)))
    if any(rc != 0 for rc in rcs):
        raise OracleError("repack_w8")
    return w8, sc


def quantize_a8(a: np.ndarray, k_pad: int | None = None):
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    k_pad = k if k_pad is None else k_pad
    a8 = np.empty((m, k_pad), np.int8)
    sc = np.empty(m, np.float32)
    if lib().or_quantize_a8(_p(a, _f32p), m, k, k_pad, _p(a8, _i8p), _p(sc, _f32p)) != 0:
        raise OracleError("quantize_a8")
    return a8, sc


def gemm_i32(a8: np.ndarray, w8: np.ndarray, threads: int = 1) -> np.ndarray:
    a8 = np.ascontiguousarray(a8)
    w8 = np.ascontiguousarray(w8)
    m, k = a8.shape
    n = w8.shape[0]
    assert w8.shape[1] == k
    c = np.empty((m, n), np.int32)
    lib().or_gemm_i32(_p(a8, _i8p), _p(w8, _i8p), m, n, k, _p(c, _i32p), threads)
    return c


def rescale(c: np.ndarray, a_scales: np.ndarray, w_scales: np.ndarray, neon: bool = False) -> np.ndarray:
    """(f32(c) * a) * w; neon=True gives the aarch64 prompt-path order (c * w) * a."""
    m, n = c.shape
    out = np.empty((m, n), np.float32)
    (lib().or_rescale_neon if neon else lib().or_rescale)(_p(np.ascontiguousarray(c), _i32p), _p(np.ascontiguousarray(a_scales, np.float32), _f32p),
                     _p(np.ascontiguousarray(w_scales, np.float32), _f32p), m, n, _p(out, _f32p))
    return out


def matmul_q_w8a8(kind: int, blocks: np.ndarray, a: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    if lib().or_matmul_q_w8a8(kind, _p(blocks, _u8p), blocks.nbytes, _p(a, _f32p), m, k, n, _p(out, _f32p),
                              threads) != 0:
        raise OracleError("matmul_q_w8a8")
    return out


FNV_OFFSET = 14695981039346656037


def fnv1a64(data: bytes, h: int = FNV_OFFSET) -> int:
    buf = np.frombuffer(bytes(data), np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    return int(lib().or_fnv1a64(h, _p(buf, _u8p), len(data)))


def source_fingerprint(source: np.ndarray) -> int:
    """W8 sidecar provenance fingerprint (ggml-rocknpu.cpp:123-146)."""
    src = np.ascontiguousarray(source).view(np.uint8).reshape(-1)
    buf = src if src.size else np.zeros(1, np.uint8)
    return int(lib().or_source_fingerprint(_p(buf, _u8p), src.size))


def hilo_stack(a: np.ndarray) -> np.ndarray:
    """[a; residual(a)] as 2m rows (lib.rs:2045-2071)."""
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    st = np.empty((2 * m, k), np.float32)
    if lib().or_hilo_stack(_p(a, _f32p), m, k, _p(st, _f32p)) != 0:
        raise OracleError("hilo_stack")
    return st


def hilo_sum(stacked_out: np.ndarray) -> np.ndarray:
    """Sum of the two output halves of a [2m, n] result (lib.rs:2073-2082)."""
    st = np.ascontiguousarray(stacked_out, np.float32)
    m = st.shape[0] // 2
    out = np.empty((m,) + st.shape[1:], np.float32)
    lib().or_hilo_sum(_p(out, _f32p), _p(st, _f32p), out.size)
    return out


def matmul_q_hilo(kind: int, blocks: np.ndarray, a: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    """The prompt-path W8A8 route with the two-part activation encoding."""
    return hilo_sum(matmul_q_w8a8(kind, blocks, hilo_stack(a), n, threads=threads))


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    out = np.empty((m, (k // QK) * Q8K_BYTES), np.uint8)
    for r in range(m):
        lib().or_quantize_row_q8_k(_p(x[r], _f32p), k, _p(out[r], _u8p))
    return out


def gemv_q8_k(kind: int, w: np.ndarray, k: int, n: int, q8k: np.ndarray, threads: int = 1) -> np.ndarray:
    q8k = np.ascontiguousarray(q8k)
    m = q8k.shape[0]
    out = np.empty((m, n), np.float32)
    if lib().or_gemv_q8_k(kind, _p(w, _u8p), k, n, _p(q8k, _u8p), m, _p(out, _f32p), threads) != 0:
        raise OracleError("gemv_q8_k")
    return out


def gemv_block_sums(kind: int, w: np.ndarray, k: int, n: int, q8k_row: np.ndarray):
    nb = k // QK
    isum = np.empty((n, nb), np.int32)
    msum = np.empty((n, nb), np.int32)
    mag = np.empty(n, np.float64)
    q8k_row = np.ascontiguousarray(q8k_row)
    if lib().or_gemv_block_sums(kind, _p(w, _u8p), k, n, _p(q8k_row, _u8p), _p(isum, _i32p), _p(msum, _i32p),
                                _p(mag, _f64p)) != 0:
        raise OracleError("gemv_block_sums")
    return isum, msum, mag
