"""Tile choice of the W8A8 GEMM (rocknpu_hip_gemm_route, include/rocknpu_hip.h)
on the CPU: the route of every shape whose measured times the rules rest on,
and the invariants the rules keep over a grid of shapes. Host logic only; the
choice never changes the (exact) results, which the GPU tests check per route."""
import ctypes
import itertools

import pytest

from rocknpu_amd import _lib

CUS = 256  # MI355X


def route(m, n, k, cus=CUS):
    bm, bn, st = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.load().rocknpu_hip_gemm_route(m, n, k, cus, ctypes.byref(bm), ctypes.byref(bn), ctypes.byref(st))
    assert rc == 0
    return bm.value, bn.value, st.value


def tiles(m, n, bm, bn):
    return -(-m // bm) * -(-n // bn)


@pytest.mark.parametrize("m,n,k,expect", [
    # weight-streaming kernel while m * k fits its 112 KiB of LDS
    (1, 5632, 2048, (0, 0, 0)),
    (16, 17, 7168, (0, 0, 0)),
    (16, 40, 7232, (64, 32, 4)),
    # up to 64 rows
    (24, 5632, 2048, (64, 32, 4)),
    (40, 11264, 2048, (64, 64, 4)),      # 64x32 tiles do not fit, 64x64 do
    (32, 11264, 2048, (32, 64, 4)),      # up to 32 rows: 32x64 tiles (8.6 -> 8.2 us)
    (32, 28672, 4096, (32, 64, 4)),      # 31.8 -> 28.4 us
    (17, 32000, 2048, (32, 64, 4)),      # 18.4 -> 15.7 us
    (32, 28672, 4160, (64, 64, 4)),      # K % 128 != 0: no 32-row tiles
    (64, 28672, 4096, (64, 64, 4)),      # 448 64x64 tiles, two per CU: 34.5 -> 31.1 us
    (64, 32000, 2048, (64, 64, 2)),      # 500 tiles, more than 1.75 per CU: 17.9 against 19.2 us
    (64, 128256, 2048, (64, 64, 2)),     # 77.3 -> 62.0 us
    (64, 16500, 128, (64, 64, 4)),
    # up to 128 rows
    (128, 5632, 2048, (64, 64, 4)),      # the 5632 x 2048 Q4_K weight at 128 tokens
    (128, 2048, 2048, (64, 32, 4)),
    (128, 11264, 2048, (128, 64, 4)),    # 64x64 tiles do not fit, 128x64 do
    (128, 32000, 2048, (128, 128, 3)),   # neither 64x64 nor 128x64 fit, 128x128 do (TinyLlama head)
    (100, 16500, 128, (64, 64, 2)),
    # up to 256 rows
    (256, 11264, 2048, (128, 128, 3)),
    (256, 14336, 4096, (128, 128, 3)),
    (200, 2048, 2048, (64, 32, 4)),
    (250, 16500, 128, (256, 128, 3)),    # 128x128 tiles do not fit: the longer products' rules
    (256, 28672, 2048, (256, 128, 3)),   # 40.8 -> 22.6 us against 128x64 two per CU
    (256, 32000, 2048, (256, 128, 3)),   # 42.9 -> 24.5 us
    (256, 128256, 2048, (256, 256, 2)),  # 138.7 -> 90.5 us
    (128, 128256, 2048, (128, 128, 2)),  # the Llama-3.2-1B head: 95.6 -> 71.3 us against 64x64
    # above: one 256 x 256 tile per CU or more
    (4096, 14336, 4096, (256, 256, 2)),  # 4 rounds against 7 x 0.61 of 256x128
    (8192, 8192, 8192, (256, 256, 2)),
    (2048, 11264, 2048, (256, 128, 3)),  # 3 x 0.61 rounds against 2
    # above: 128 x 128 tiles that do not fit
    (512, 11264, 2048, (256, 128, 3)),   # 256x128 tiles fit
    (768, 8192, 2048, (256, 128, 3)),
    (1024, 14336, 4096, (256, 256, 2)),  # 1 x 1.38 rounds against 2 of 128x128 two per CU
    (520, 16500, 2048, (256, 256, 2)),
    (640, 11264, 2048, (128, 128, 2)),   # 1 x 1.38 against 1
    # above: the filling choice
    (512, 2048, 5632, (64, 64, 4)),
    (512, 1024, 4096, (64, 32, 4)),
    (512, 2560, 2048, (128, 64, 4)),
    (1024, 2560, 4096, (128, 128, 3)),   # 128x64 tiles would need two per CU
    (2048, 2048, 4096, (128, 128, 3)),
])
def test_measured_routes(m, n, k, expect):
    assert route(m, n, k) == expect


def test_invariants_over_a_grid():
    ms = (1, 8, 16, 17, 40, 64, 65, 100, 128, 129, 200, 256, 257, 384, 512, 640, 768, 1024, 1536, 2048, 4096)
    ns = (16, 100, 1024, 2048, 2560, 4096, 5632, 8192, 11264, 14336, 16384, 28672, 32000)
    ks = (64, 256, 2048, 5632, 7232, 14336)
    for m, n, k in itertools.product(ms, ns, ks):
        bm, bn, st = route(m, n, k)
        if bm == 0:
            assert m <= 16 and m * k <= 112 * 1024
            continue
        assert not (m <= 16 and m * k <= 112 * 1024)
        assert (bm, bn) in {(32, 64), (64, 32), (64, 64), (128, 64), (128, 128), (256, 128), (256, 256)}
        t = tiles(m, n, bm, bn)
        # tile height follows M: 32 or 64 rows up to 64, at most 128 up to 128, 256 from 129 rows
        # only where 128x128 tiles do not fit
        assert bm in (32, 64) or m > 64
        assert bm <= 128 or m > 256 or (m > 128 and tiles(m, n, 128, 128) > CUS)
        if (bm, bn) == (32, 64):
            # up to 32 rows where 64x32 tiles do not fit, 128-byte stages only
            assert m <= 32 and k % 128 == 0 and st == 4 and tiles(m, n, 64, 32) > CUS
        elif m <= 64 and (bm, bn) == (64, 64):
            # four stages while at most 1.75 per CU
            assert (st == 4) == (4 * t <= 7 * CUS), (m, n, k, st)
        elif bm <= 128 and (bm, bn) != (128, 128):
            # two stages exactly when the tiles outnumber the CUs (two per CU)
            assert (st == 2) == (t > CUS), (m, n, k, bm, bn, st)
            assert st in (2, 4)
        if (bm, bn) == (128, 128):
            assert (st == 3 and t <= CUS) or (st == 2 and t > CUS), (m, n, k, st)
        if (bm, bn) == (256, 128):
            assert st == 3
        if (bm, bn) == (256, 256):
            assert st == 2


def test_fewer_cus_and_bad_arguments():
    # on a part with fewer CUs the one-round rules move accordingly
    assert route(128, 11264, 2048, cus=256) == (128, 64, 4)
    assert route(128, 11264, 2048, cus=128) == (64, 64, 2)
    out = [ctypes.c_int() for _ in range(3)]
    lib = _lib.load()
    ptrs = [ctypes.byref(o) for o in out]
    assert lib.rocknpu_hip_gemm_route(0, 64, 64, CUS, *ptrs) == -1
    assert lib.rocknpu_hip_gemm_route(4, 64, 100, CUS, *ptrs) == -1  # k_pad % 64 != 0
    assert lib.rocknpu_hip_gemm_route(4, 64, 64, CUS, None, ptrs[1], ptrs[2]) == -1


def workspace(m, n, k, cus=CUS):
    nb, sp = ctypes.c_size_t(), ctypes.c_int()
    assert _lib.load().rocknpu_hip_gemm_workspace(m, n, k, cus, ctypes.byref(nb), ctypes.byref(sp)) == 0
    return nb.value, sp.value


@pytest.mark.parametrize("m,n,k,splits", [
    # 64 x 32 tiles on half the CUs, long K: split so the units fill the CUs
    (128, 2048, 4096, 2),    # 10.9 -> 10.2 us
    (128, 2048, 5632, 2),    # TinyLlama down: 13.6 -> 11.7 us
    (128, 2048, 8192, 2),    # Llama-3.2-1B down: 18.0 -> 13.8 us
    (64, 4096, 14336, 2),
    (32, 2048, 5632, 3),     # 32 tiles: at most three splits (13.2 -> 10.5 us)
    (32, 2560, 4096, 3),     # 9.8 us against 10.6 in four
    (32, 2048, 8192, 3),
    (128, 2048, 2048, 1),    # 16 stages: 6.6 us unsplit against 8.0 in two (TinyLlama o at 128 tokens)
    (32, 2560, 2048, 1),     # 7.3 against 8.4
    # measured slower split, or not under-filled: unsplit
    (128, 5632, 2048, 1),    # 176 64 x 64 tiles (8.4 against 12.0 us split)
    (128, 2560, 2048, 1),    # 160 tiles: more than half the CUs
    (1024, 8192, 4096, 1),   # 256 x 256 tiles (58.5 against 63.9 us split)
    (512, 11264, 2048, 1),
    (4096, 14336, 4096, 1),
    (128, 2048, 256, 1),     # two stages: nothing to split
    (8, 2048, 8192, 1),      # the weight-streaming kernel
])
def test_split_rule(m, n, k, splits):
    nb, sp = workspace(m, n, k)
    assert sp == splits
    bm, bn, _ = route(m, n, k)
    if sp == 1:
        assert nb == 0
    else:
        t = tiles(m, n, bm, bn)
        # the fixed 16 KiB counter block, then splits x bm x bn int32 per tile,
        # then one 4-byte stamp per (tile, split) rounded up to 256 bytes
        assert nb == 16384 + t * sp * bm * bn * 4 + -(-t * sp * 4 // 256) * 256


def test_split_invariants_over_a_grid():
    ms = (1, 16, 17, 32, 64, 100, 128, 200, 256, 512, 1024, 4096)
    ns = (16, 100, 1024, 2048, 2560, 4096, 5632, 11264, 32000)
    ks = (64, 256, 1024, 2048, 5632, 8192, 14336)
    for m, n, k in itertools.product(ms, ns, ks):
        nb, sp = workspace(m, n, k)
        bm, bn, _ = route(m, n, k)
        if sp == 1:
            assert nb == 0
            continue
        t = tiles(m, n, bm, bn)
        stages = k // 128 if k % 128 == 0 else k // 64
        assert bm * bn <= 64 * 64 and 2 * t <= CUS, (m, n, k)
        assert 2 <= sp <= 4 and t * sp <= CUS and stages // sp >= 8, (m, n, k, sp)
        # the no-allocation entry's fixed split workspace holds every routed split on 256 CUs
        assert nb <= (4 << 20) + 16384 + 1024, (m, n, k, nb)


def test_workspace_and_tile_bad_arguments():
    lib = _lib.load()
    nb, sp = ctypes.c_size_t(), ctypes.c_int()
    assert lib.rocknpu_hip_gemm_workspace(0, 64, 64, CUS, ctypes.byref(nb), ctypes.byref(sp)) == -1
    assert lib.rocknpu_hip_gemm_workspace(4, 64, 100, CUS, ctypes.byref(nb), ctypes.byref(sp)) == -1
    assert lib.rocknpu_hip_gemm_workspace(4, 64, 64, CUS, None, ctypes.byref(sp)) == -1
    # every check below fails on the host, before any GPU call
    p = ctypes.c_void_p(1 << 20)  # never dereferenced
    args = (p, p, p, p, 128, 2048, 2048, p, 2048, None)
    assert lib.rocknpu_hip_gemm_w8a8_tile(64, 48, 4, 1, *args, None, 0, None) == -1   # no such tile
    assert lib.rocknpu_hip_gemm_w8a8_tile(64, 64, 3, 1, *args, None, 0, None) == -1   # no such stage count
    assert lib.rocknpu_hip_gemm_w8a8_tile(64, 32, 4, 0, *args, None, 0, None) == -1   # splits < 1
    assert lib.rocknpu_hip_gemm_w8a8_tile(64, 32, 4, 2, *args, None, 0, None) == -1   # split without workspace
    units = (128 // 64) * (2048 // 32) * 2
    small = 16384 + units * 64 * 32 * 4 + units * 4 - 4  # four bytes short
    assert lib.rocknpu_hip_gemm_w8a8_tile(64, 32, 4, 2, *args, p, small, None) == -1
    assert lib.rocknpu_hip_gemm_w8a8_ws(*args, ctypes.c_void_p((1 << 20) + 16), 4096, None) == -1  # unaligned
    assert lib.rocknpu_hip_gemm_w8a8_ws(*args, None, 4096, None) == -1


def column_split(m, n, k, cus=CUS):
    n0 = ctypes.c_size_t()
    assert _lib.load().rocknpu_hip_gemm_column_split(m, n, k, cus, ctypes.byref(n0)) == 0
    return n0.value


@pytest.mark.parametrize("m,n,k,expect", [
    # whole rounds of 256 x 256 tiles plus a last round at most half full: the
    # whole rounds' columns as one launch, the rest as a second
    (4096, 14336, 4096, 12288),   # 896 tiles: 3 rounds + 128 (Llama-3-8B gate/up at 4096 tokens)
    (1536, 11264, 4096, 10752),   # 264 tiles: 1 round + 8
    (1536, 14336, 2048, 10752),   # 336 tiles: 1 round + 80
    (768, 28672, 2048, 21760),    # 336 tiles
    (4096, 5632, 4096, 4096),     # 352 tiles: 1 round + 96
    (2048, 28672, 4096, 24576),   # 896 tiles: 3 rounds + 128, exactly half full
    # one launch: the last round more than half full, no whole round, whole
    # rounds only, or M <= 256
    (1024, 28672, 4096, 0),       # 448 tiles: 1 round + 192
    (4096, 11264, 2048, 0),       # 704 tiles: 2 rounds + 192
    (2048, 5632, 4096, 0),        # 176 tiles: less than a round
    (4096, 28672, 4096, 0),       # 1792 tiles: 7 whole rounds
    (256, 28672, 2048, 0),
    (4096, 256, 4096, 0),
])
def test_column_split(m, n, k, expect):
    assert column_split(m, n, k) == expect


def test_column_split_invariants():
    for m, n in itertools.product((257, 512, 1000, 1536, 2048, 3000, 4096, 8192), range(256, 40000, 768)):
        n0 = column_split(m, n, 2048)
        t = tiles(m, n, 256, 256)
        if n0 == 0:
            continue
        assert n0 % 256 == 0 and 0 < n0 < n
        main = tiles(m, n0, 256, 256)
        assert main % CUS == 0 or main <= CUS * (t // CUS)    # whole rounds' worth at most
        assert t // CUS >= 1 and 2 * (t - CUS * (t // CUS)) <= CUS
    lib = _lib.load()
    n0 = ctypes.c_size_t()
    assert lib.rocknpu_hip_gemm_column_split(0, 64, 64, CUS, ctypes.byref(n0)) == -1
    assert lib.rocknpu_hip_gemm_column_split(4, 64, 100, CUS, ctypes.byref(n0)) == -1
    assert lib.rocknpu_hip_gemm_column_split(4096, 14336, 4096, CUS, None) == -1
