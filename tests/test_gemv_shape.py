"""Launch shape of the decode GEMV (rocknpu_hip_gemv_shape, include/rocknpu_hip.h)
on the CPU: the shapes the TinyLlama and Llama-3-8B projections run with (the
kernels listed in profiles/bench_kernel_stats.md), and the invariants of the
choice. Host logic only; the GPU tests check every shape's results."""
import ctypes

import pytest

from rocknpu_amd import _lib

CUS = 256  # MI355X


def shape(kind, m, k, ns, fused=True, cus=CUS):
    arr = (ctypes.c_size_t * len(ns))(*ns)
    mf, lanes, waves = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.load().rocknpu_hip_gemv_shape(kind, m, k, arr, len(ns), 1 if fused else 0, cus, ctypes.byref(mf),
                                            ctypes.byref(lanes), ctypes.byref(waves))
    assert rc == 0
    if mf.value == 2:
        return ("stream", waves.value)
    return ("mfma",) if mf.value else (lanes.value, waves.value)


def slots_log2(nb, slots=8):
    """Block slots per row (log2) of gemv.hip's slots_per_row_log2."""
    lg = 0
    while (2 << lg) <= slots and (2 << lg) <= nb:
        lg += 1
    while lg > 0:
        g = 1 << lg
        it = (nb + g - 1) // g
        if nb * 100 >= 85 * g * it:
            break
        lg -= 1
    return lg


@pytest.mark.parametrize("kind,m,k,ns,expect", [
    # TinyLlama-1.1B, one token: q/k/v, o, gate+up (Q4_K), down (Q6_K)
    (4, 1, 2048, [2048, 256, 256], (4, 8)),
    (4, 1, 2048, [2048], (8, 8)),
    (4, 1, 2048, [5632, 5632], (4, 16)),   # a wider L with 16 waves fills every CU
    (6, 1, 5632, [2048], ("stream", 8)),
    # four tokens: Q4_K on the matrix cores, Q6_K down on the LDS stream
    (4, 4, 2048, [2048], ("mfma",)),
    (4, 4, 2048, [5632, 5632], ("mfma",)),
    (6, 4, 5632, [2048], ("stream", 8)),
    # Llama-3-8B, one token: gate+up (Q4_K), down (Q6_K on the stream, 8 waves of two rows)
    (4, 1, 4096, [14336, 14336], (4, 8)),
    (6, 1, 14336, [4096], ("stream", 8)),
    # Llama-3-8B down at 2-4 tokens: 16 stream waves
    (6, 4, 14336, [4096], ("stream", 16)),
    (6, 3, 14336, [4096], ("stream", 16)),
    (6, 2, 14336, [4096], ("stream", 16)),
    # rows that do not split into 8 block slots stay on the lane-per-block kernel
    (6, 1, 2560, [2048], (8, 16)),
    # Q4_K from 3 rows, Q6_K from 5 rows on the matrix cores
    (4, 2, 2048, [2048], (8, 8)),
    (4, 3, 2048, [2048], ("mfma",)),
    (6, 5, 5632, [2048], ("mfma",)),
])
def test_projection_shapes(kind, m, k, ns, expect):
    assert shape(kind, m, k, ns) == expect


def test_invariants():
    for kind in (4, 6):
        for m in range(1, 9):
            for k in (256, 2048, 4096, 5632, 14336):
                for ns in ([16], [256], [2048], [2048, 256, 256], [5632, 5632], [14336, 14336], [32000]):
                    for fused in (True, False):
                        got = shape(kind, m, k, ns, fused)
                        nb = k // 256
                        if kind == 6 and m <= 4 and nb <= 64 and slots_log2(nb) == 3:
                            assert got == ("stream", 16 if m > 1 and sum(ns) >= 16 * CUS else 8), (m, k, ns, got)
                            continue
                        mfma = m >= 3 if kind == 4 else (m >= 5 or (m >= 3 and sum(ns) >= 16 * CUS))
                        assert (got == ("mfma",)) == mfma, (kind, m, k, ns, got)
                        if mfma:
                            continue
                        lanes, waves = got
                        assert lanes in (2, 4, 8) and waves in (8, 16)
                        if not fused:
                            assert waves == 16  # 8-wave workgroups serve fused launches only


def test_bad_arguments():
    lib = _lib.load()
    arr = (ctypes.c_size_t * 1)(2048)
    out = [ctypes.c_int() for _ in range(3)]
    ptrs = [ctypes.byref(o) for o in out]
    assert lib.rocknpu_hip_gemv_shape(5, 1, 2048, arr, 1, 1, CUS, *ptrs) == -1     # Q5_K has no GEMV
    assert lib.rocknpu_hip_gemv_shape(4, 1, 256 * 1000, arr, 1, 1, CUS, *ptrs) == -1  # rows beyond the LDS
    assert lib.rocknpu_hip_gemv_shape(4, 1, 2000, arr, 1, 1, CUS, *ptrs) == -1     # K % 256 != 0
    assert lib.rocknpu_hip_gemv_shape(4, 1, 2048, arr, 5, 1, CUS, *ptrs) == -1     # more than 4 members
    assert lib.rocknpu_hip_gemv_shape(4, 1, 2048, None, 1, 1, CUS, *ptrs) == -1
