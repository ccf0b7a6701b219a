"""The oracle reproduces the golden fixtures (tests/golden, written by
make_golden.py from the reference's known-answer patterns and the independent
numpy restatement)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLD / f"{name}.npz", allow_pickle=False)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["rounding_kat", "max_abs_kat"])
def test_golden_quantize_symmetric(name):
    f = _load(name)
    q, s = orc.quantize_symmetric_row(f["x"])
    assert np.array_equal(q, f["q"]) and np.float32(s) == f["scale"][0]


def test_golden_gemm_kats():
    f = _load("gemm_kats")
    for name in ("m1", "m1_neg", "mtile_uniform", "ksplit"):
        c = orc.gemm_i32(f[f"{name}_a"], f[f"{name}_w"], threads=4)
        assert np.array_equal(c, f[f"{name}_c"]), name
        out = orc.rescale(c, f[f"{name}_as"], f[f"{name}_ws"])
        assert np.array_equal(_bits(out), _bits(f[f"{name}_out"])), name


@pytest.mark.parametrize("kind", [4, 6])
def test_golden_repack(kind):
    f = _load(f"repack_q{kind}k")
    w8, sc = orc.repack_w8(kind, f["blocks"], int(f["k"]), int(f["n"]))
    assert np.array_equal(w8, f["w8"]) and np.array_equal(_bits(sc), _bits(f["scales"]))


def test_golden_quantize_a8():
    f = _load("quantize_a8")
    a8, sc = orc.quantize_a8(f["a"], int(f["k_pad"]))
    assert np.array_equal(a8, f["a8"]) and np.array_equal(_bits(sc), _bits(f["scales"]))


def test_golden_q8_k():
    f = _load("q8_k")
    assert np.array_equal(orc.quantize_q8_k(f["x"]), f["q8k"])


@pytest.mark.parametrize("kind", [4, 6])
def test_golden_gemv(kind):
    f = _load(f"gemv_q{kind}k")
    k, n = int(f["k"]), int(f["n"])
    out = orc.gemv_q8_k(kind, f["w"], k, n, f["q8k"])
    for mi in range(f["q8k"].shape[0]):
        isum, msum, _ = orc.gemv_block_sums(kind, f["w"], k, n, f["q8k"][mi])
        assert np.array_equal(isum, f["isum"][mi]) and np.array_equal(msum, f["msum"][mi])
        assert np.all(np.abs(out[mi].astype(np.float64) - f["y"][mi]) <= 1e-5 * f["mag"][mi] + 1e-30)


def test_golden_q5_k_high_bits():
    """Each qh bit alone moves exactly one value by +16, at the position
    dequantize_row_q5_K assigns it: bit 2j -> value l of 64-chunk j, bit 2j + 1
    -> value 32 + l. The oracle's dequant and repack reproduce the closed form."""
    f = _load("repack_q5k_bits")
    n = int(f["n"])
    y = orc.dequant_rows(5, f["blocks"], 256, n)
    assert np.array_equal(_bits(y), _bits(f["y"]))
    w8, sc = orc.repack_w8(5, f["blocks"], 256, n)
    assert np.array_equal(w8, f["w8"]) and np.array_equal(_bits(sc), _bits(f["scales"]))
    # a restatement with the two bits of a chunk swapped fails the closed form
    b = f["blocks"].reshape(n, 176)
    qh = b[:, 16:48].astype(np.int32)
    qs = b[:, 48:].astype(np.int32).reshape(n, 4, 32)
    swapped = np.empty((n, 256), np.float32)
    for j in range(4):
        swapped[:, 64 * j:64 * j + 32] = qs[:, j] % 16 + 16 * ((qh >> (2 * j + 1)) & 1)
        swapped[:, 64 * j + 32:64 * j + 64] = qs[:, j] // 16 + 16 * ((qh >> (2 * j)) & 1)
    assert not np.array_equal(swapped, f["y"])
    # and so does reading bit j of qh[l] for chunk j (one bit per chunk)
    one_bit = np.empty((n, 256), np.float32)
    for j in range(4):
        one_bit[:, 64 * j:64 * j + 32] = qs[:, j] % 16 + 16 * ((qh >> j) & 1)
        one_bit[:, 64 * j + 32:64 * j + 64] = qs[:, j] // 16 + 16 * ((qh >> (j + 4)) & 1)
    assert not np.array_equal(one_bit, f["y"])


def test_golden_q8_k_half_even_ties():
    """iscale = 1.0 exactly, so every +-(j + 1/2) is an exact tie: ggml's
    nearest_int gives the even neighbour. A planted roundf (half away from zero,
    the W8A8 quantiser's rule) fails the fixture."""
    f = _load("q8_k_ties")
    got = orc.quantize_q8_k(f["x"])[0]
    assert np.array_equal(got[:292], f["q8k_block0"])
    x = f["x"][0, :256]
    q = np.frombuffer(f["q8k_block0"][4:260].tobytes(), np.int8).astype(np.int32)
    assert np.frombuffer(f["q8k_block0"][0:4].tobytes(), np.float32)[0] == 1.0
    away = np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))
    assert not np.array_equal(away.astype(np.int32), q)
    # the rest of the row is ordinary data, checked against the numpy restatement
    from . import np_ref
    assert np.array_equal(got[292:], np_ref.pack_q8_k(*np_ref.quantize_q8_k(f["x"][0, 256:])))
