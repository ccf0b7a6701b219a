"""The C-ABI library on the CPU: it loads, exports every symbol include/*.h
declares, and its argument guards answer before any device work (no compute
calls here)."""
import ctypes
import re

import numpy as np
import pytest

from rocknpu_amd import _lib

from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(rocknpu_\w+)\s*\(", text))
    return names


def test_headers_declare_the_reference_abi():
    ref_abi = {
        "rocknpu_device_count", "rocknpu_context_create", "rocknpu_context_decode_cache_stats",
        "rocknpu_context_destroy", "rocknpu_context_set_overlap", "rocknpu_matmul_q_concat_f32_f32_mtile",
        "rocknpu_mtile_release", "rocknpu_prewarm_quantized_m16", "rocknpu_matmul_f16_f32_f32",
        "rocknpu_matmul_w8a8_f32_f32_m1", "rocknpu_matmul_w8a8_f32_f32_m16",
        "rocknpu_matmul_w8a8_f32_f32_m1_nsplit", "rocknpu_matmul_w8a8_swiglu_down_f32",
        "rocknpu_matmul_w8a8_pair_f32_f32_m1", "rocknpu_matmul_q_pair_f32_f32_mtile",
        "rocknpu_matmul_w8a8_triple_f32_f32_m1", "rocknpu_matmul_q_pair_f32_f32_m1",
        "rocknpu_matmul_q_triple_f32_f32_m1", "rocknpu_matmul_q4_k_f32_f32", "rocknpu_matmul_q5_k_f32_f32",
        "rocknpu_matmul_q6_k_f32_f32",
    }
    assert ref_abi <= _declared_symbols()  # the 21 symbols of crates/rocknpu-capi/include/rocknpu.h


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert declared == set(_lib.SIGNATURES), "ctypes table out of sync with the headers"


def test_library_is_gfx950_only():
    data = _lib.LIB_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in data


def test_null_context_guards():
    lib = _lib.load()
    # crates/rocknpu-capi/src/lib.rs:5791-5806: a null context is rejected before any pointer access
    assert lib.rocknpu_matmul_f16_f32_f32(None, None, None, None, 4, 32, 16) == -1
    assert lib.rocknpu_matmul_q4_k_f32_f32(None, None, 0, None, None, 1, 256, 1) == -1
    assert lib.rocknpu_matmul_q6_k_f32_f32(None, None, 0, None, None, 1, 256, 1) == -1
    assert lib.rocknpu_matmul_q5_k_f32_f32(None, None, 0, None, None, 2, 256, 1) == -1
    assert lib.rocknpu_matmul_w8a8_f32_f32_m1(None, None, None, None, None, 64, 32) == -1
    assert lib.rocknpu_mtile_release(None, 1, None) == -1
    assert lib.rocknpu_context_set_overlap(None, None, None) == -1
    assert lib.rocknpu_context_decode_cache_stats(None, None) == -1
    assert lib.rocknpu_matmul_q_q8k_f32_f32(None, 4, None, 0, None, None, 1, 256, 1) == -1
    lib.rocknpu_context_destroy(None)  # no-op


def test_launch_layer_rejects_bad_shapes_before_launch():
    lib = _lib.load()
    buf = np.zeros(4096, np.uint8)
    p = ctypes.c_void_p(buf.ctypes.data)
    # k not a multiple of 256, wrong byte count, unaligned k_pad, bad kind
    assert lib.rocknpu_hip_repack_w8(4, p, 144, 100, 1, 128, p, p, None) == -1
    assert lib.rocknpu_hip_repack_w8(4, p, 143, 256, 1, 256, p, p, None) == -1
    assert lib.rocknpu_hip_repack_w8(4, p, 144, 256, 1, 260, p, p, None) == -1
    assert lib.rocknpu_hip_repack_w8(7, p, 144, 256, 1, 256, p, p, None) == -1
    assert lib.rocknpu_hip_gemm_w8a8(p, p, p, p, 4, 4, 100, p, 4, None, None) == -1
    # int32 sums are exact only while 127 * 127 * K < 2^31: K = 133120 is the largest multiple of 64
    assert 127 * 127 * 133120 < 2**31 <= 127 * 127 * 133184
    assert lib.rocknpu_hip_gemm_w8a8(p, p, p, p, 4, 4, 133184, p, 4, None, None) == -1
    assert lib.rocknpu_hip_quantize_q8_k(p, 1, 100, 100, p, None) == -1
    assert lib.rocknpu_hip_gemv_q8_k(5, p, 144, 256, 1, p, 1, p, 1, None, None, None) == -1
    assert lib.rocknpu_hip_gemv_q8_k(4, p, 144, 256, 1, p, 1, p, 1, p, None, None) == -1


def test_no_device_means_no_context():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = _lib.load()
    assert lib.rocknpu_device_count() == 0
    assert not lib.rocknpu_context_create()


def test_gemv_stall_report_host_side():
    """The decode GEMV's stall report before any launch: the flag reads 0 (no
    fused launch has allocated it), the test hook refuses a negative count and
    accepts 0 (normal launches)."""
    lib = _lib.load()
    assert lib.rocknpu_hip_gemv_take_stall() == 0
    assert lib.rocknpu_hip_gemv_test_stall(-1) == -1
    assert lib.rocknpu_hip_gemv_test_stall(0) == 0
    assert lib.rocknpu_hip_gemv_take_stall() == 0


def test_tiled_decode_layout_host_side():
    """Bytes of the tiled decode copies (whole 16-row tiles of k/256 blocks), and
    the tiled entries' argument checks, all answered on the host."""
    lib = _lib.load()
    assert lib.rocknpu_hip_gemv_tiled_bytes(4, 2048, 2048) == 2048 * 8 * 144
    assert lib.rocknpu_hip_gemv_tiled_bytes(6, 5632, 2048) == 2048 * 22 * 210
    assert lib.rocknpu_hip_gemv_tiled_bytes(4, 2048, 17) == 32 * 8 * 144   # ragged rows pad to a tile
    assert lib.rocknpu_hip_gemv_tiled_bytes(6, 256, 1) == 16 * 210
    assert lib.rocknpu_hip_gemv_tiled_bytes(5, 2048, 16) == 0               # no Q5_K GEMV
    assert lib.rocknpu_hip_gemv_tiled_bytes(4, 100, 16) == 0                # K not a multiple of 256
    assert lib.rocknpu_hip_gemv_tiled_bytes(4, 256, 0) == 0
    p = ctypes.c_void_p(1 << 20)  # never dereferenced
    raw = 16 * 144
    tb = lib.rocknpu_hip_gemv_tiled_bytes(4, 256, 16)
    assert lib.rocknpu_hip_gemv_tile_weights(4, p, raw, 256, 16, p, tb - 1, None) == -1     # copy too small
    assert lib.rocknpu_hip_gemv_tile_weights(4, p, raw - 144, 256, 16, p, tb, None) == -1   # raw bytes != n rows
    assert lib.rocknpu_hip_gemv_tile_weights(4, p, raw, 256, 16, ctypes.c_void_p((1 << 20) + 8), tb, None) == -1
    assert lib.rocknpu_hip_gemv_tile_weights(4, None, raw, 256, 16, p, tb, None) == -1
    out = ctypes.c_void_p(1 << 21)
    assert lib.rocknpu_hip_gemv_q8_k_tiled(4, p, 17 * 144, 256, 17, p, 1, out, 17, None, 0, None) == -1  # raw size, not tiled
    assert lib.rocknpu_hip_gemv_q8_k_tiled(4, p, tb, 256, 16, p, 1, out, 8, None, 0, None) == -1     # ldo < n
    w_arr = (ctypes.c_void_p * 1)(1 << 20)
    b_arr = (ctypes.c_size_t * 1)(tb)
    n_arr = (ctypes.c_size_t * 1)(16)
    o_arr = (ctypes.c_void_p * 1)(1 << 21)
    l_arr = (ctypes.c_size_t * 1)(16)
    assert lib.rocknpu_hip_gemv_q_f32_tiled(4, 1, w_arr, b_arr, n_arr, 256, p, 255, 1, o_arr, l_arr, None, 0, None) == -1
    assert lib.rocknpu_hip_gemv_q_f32_tiled(4, 5, w_arr, b_arr, n_arr, 256, p, 256, 1, o_arr, l_arr, None, 0, None) == -1
    b_arr[0], n_arr[0], l_arr[0] = 17 * 144, 17, 17  # raw size of 17 rows, not the tiled 32
    assert lib.rocknpu_hip_gemv_q_f32_tiled(4, 1, w_arr, b_arr, n_arr, 256, p, 256, 1, o_arr, l_arr, None, 0, None) == -1


@pytest.mark.parametrize("kind,m,k,tiled", [
    (4, 2, 2048, 1), (6, 4, 5632, 1), (4, 8, 256, 1),       # from two rows: always the tiled copy
    (4, 1, 2048, 1), (6, 1, 2048, 1),                        # TinyLlama o / qkv / gate+up: 8 blocks, tiled
    (4, 1, 1280, 1), (6, 1, 1792, 1),                        # 5-7 blocks: tiled
    (4, 1, 2560, 1), (4, 1, 4096, 1), (6, 1, 4096, 1),       # 9-16 blocks: tiled
    (4, 1, 5632, 0), (6, 1, 5632, 0), (6, 1, 7936, 0),       # 17-31 blocks filling 8 slots (21-24, 28-31): raw
    (4, 1, 4352, 1), (6, 1, 5120, 1), (6, 1, 6656, 1),       # 17, 20 and 26 blocks (fewer slots): tiled
    (4, 1, 8192, 1), (6, 1, 14336, 1), (4, 1, 28672, 1),     # 32 and more (Q6_K up to 64): tiled
    (6, 1, 16640, 0),                                        # Q6_K beyond 64 blocks: raw
    (4, 1, 1024, 0), (6, 1, 1024, 0), (4, 1, 256, 0),        # at most 4 blocks: raw
    (5, 2, 2048, 0), (4, 1, 100, 0),                         # no Q5_K; K % 256
])
def test_tiled_rule_host_side(kind, m, k, tiled):
    assert _lib.load().rocknpu_hip_gemv_tiled_preferred(kind, m, k) == tiled


def test_tiled_split_workspace_bytes_host_side():
    """The tiled GEMV's K-split workspace: 256 bytes (the error word) and
    S - 1 8-byte slots (S ranges) per 16-row tile, lane and register row (one
    for launches of up to 4 rows, two for 5-8), sized by the call's largest
    launch; 0 where nothing splits."""
    lib = _lib.load()
    wsb = lib.rocknpu_hip_gemv_tiled_workspace_bytes
    tiles = 2048 // 16
    assert wsb(6, 4, 5632, 2048) == 256 + tiles * 64 * 8
    assert wsb(6, 2, 5632, 2048) == 256 + tiles * 64 * 8
    assert wsb(6, 8, 5632, 2048) == 256 + tiles * 64 * 2 * 3 * 8   # 5-8 rows: 4 ranges
    assert wsb(4, 5, 4352, 1000) == 256 + 63 * 64 * 2 * 3 * 8      # 17 blocks, ragged rows
    assert wsb(6, 20, 5632, 2048) == 256 + tiles * 64 * 2 * 3 * 8  # launches of 8, 8 and 4 rows
    assert wsb(6, 9, 5632, 2048) == 256 + tiles * 64 * 2 * 3 * 8   # 8 rows, then 1 (unsplit)
    assert wsb(6, 1, 5632, 2048) == 0                              # one row of 22 blocks: unsplit
    assert wsb(4, 4, 2048, 2048) == 0                              # 8 blocks
    assert wsb(4, 4, 4096, 4096) == 0                              # 16 blocks
    # 32-64 blocks from one row: 4 ranges, a tree of 3 slots
    assert wsb(6, 4, 8192, 2048) == 256 + tiles * 64 * 3 * 8       # 32 blocks: 4 ranges
    assert wsb(6, 1, 14336, 4096) == 256 + 256 * 64 * 3 * 8        # 56 blocks: 4 ranges
    assert wsb(6, 8, 14336, 4096) == 256 + 256 * 64 * 2 * 3 * 8    # 56 blocks, 8 rows
    assert wsb(4, 8, 16384, 4096) == 256 + 256 * 64 * 3 * 8        # 64 blocks: launches of 4 rows
    assert wsb(6, 4, 16640, 4096) == 0                             # 65 blocks: unsplit
    assert wsb(4, 12, 5632, 2048) == 0                             # 9-16 rows (Q4_K): unsplit
    assert wsb(5, 4, 5632, 2048) == 0 and wsb(6, 4, 5000, 2048) == 0
