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
