"""Write the golden fixtures in this directory.

Inputs are the reference's own known-answer patterns (cited per fixture) and
seeded K-quant blocks; expected outputs come from closed forms and from the
independent numpy restatement in tests/np_ref.py (never from the C oracle, so
the fixtures check the oracle and the GPU path alike).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import np_ref  # noqa: E402
from rocknpu_amd import synth  # noqa: E402


def rounding_kat() -> np.ndarray:
    # crates/rocknpu-capi/src/lib.rs:5680-5704: edge values, then 2051 LCG values
    vals = [-12.75, -7.5, -3.5, -1.5, -0.5, -0.49999997, 0.0, 0.49999997, 0.5, 1.5, 3.5, 7.5, 12.75]
    state = 0x12345678
    for _ in range(2051):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        unit = np.float32(state >> 8) / np.float32((1 << 24) - 1)
        vals.append((unit * np.float32(2.0) - np.float32(1.0)) * np.float32(17.0))
    return np.array(vals, np.float32)


def max_abs_kat() -> np.ndarray:
    # lib.rs:5714-5717
    return ((np.arange(2051) * 7919 % 65521).astype(np.float32) - np.float32(32760.0)) * np.float32(0.001)


def gemm_patterns():
    """The reference's int8 GEMM known-answer patterns with exact i32 products."""
    out = {}
    # rocket-smoke/src/bin/int8_decode_m1.rs:35-45: a[i]=((i*7+3)%9)-4, b[i]=((i*5+1)%11)-5
    k, n = 2048, 96
    i = np.arange(k)
    a = (((i * 7 + 3) % 9) - 4).astype(np.int8)[None, :]
    w = np.stack([(((i * 5 + 1 + r) % 11) - 5) for r in range(n)]).astype(np.int8)
    out["m1"] = (a, w)
    # int8_projection_profile.rs:11-22,54-56: the negated variant
    out["m1_neg"] = ((-a.astype(np.int16)).astype(np.int8), w)
    # int8_mtile.rs:28-37,71-82: input row r filled with r%5+1, weights 1 -> K*(r%5+1)
    m, k, n = 128, 2048, 64
    a = np.repeat((np.arange(m) % 5 + 1).astype(np.int8)[:, None], k, axis=1)
    out["mtile_uniform"] = (a, np.ones((n, k), np.int8))
    # int8_mtile_ksplit.rs:27: ((row*7 + kk*3 + 5) % 13) - 6
    m, k, n = 64, 6144, 32
    r, kk = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    a = (((r * 7 + kk * 3 + 5) % 13) - 6).astype(np.int8)
    rw, kw = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    w = (((rw * 5 + kw * 11 + 1) % 9) - 4).astype(np.int8)
    out["ksplit"] = (a, w)
    return out


def q5_k_single_bit_blocks():
    """Q5_K blocks with d = 1, dmin = 0, unit scales, every quant byte 0x5A
    (low nibble 10, high nibble 5) and exactly one qh bit set: block (t, l) has
    bit t of qh[l]. Per ggml dequantize_row_q5_K, value l of 64-chunk j takes
    +16 from qh[l] bit 2j (its low-nibble half) and value 32 + l from bit 2j + 1
    (its high-nibble half), so block (t, l) dequantises to the nibble values
    with +16 at position 64 (t // 2) + 32 (t % 2) + l and nowhere else."""
    blocks, expect = [], []
    for t in range(8):
        for l in range(32):
            b = np.zeros(176, np.uint8)
            b[0:2] = np.array([1.0], np.float16).view(np.uint8)
            b[4:16] = synth.pack_scales_k4(np.ones((1, 8), int), np.zeros((1, 8), int))[0]
            b[16 + l] = 1 << t
            b[48:] = 0x5A
            y = np.array([10.0 if (p % 64) < 32 else 5.0 for p in range(256)], np.float32)
            y[64 * (t // 2) + 32 * (t % 2) + l] += 16.0
            blocks.append(b)
            expect.append(y)
    return np.concatenate(blocks), np.stack(expect)


def q8_k_tie_block():
    """One 256-value block whose first largest magnitude is -127 (so iscale =
    -127 / -127 = 1.0 exactly and d = 1.0), holding +-(j + 1/2) for j = 0..126
    and a zero. ggml's nearest_int rounds half to even, so +-(j + 1/2) becomes
    +-j for even j and +-(j + 1) for odd j."""
    x = [-127.0]
    q = [-127]
    for j in range(127):
        for sign in (1.0, -1.0):
            x.append(sign * (j + 0.5))
            q.append(int(sign) * (j if j % 2 == 0 else j + 1))
    x.append(0.0)
    q.append(0)
    x, q = np.array(x, np.float32), np.array(q, np.int32)
    assert x.size == 256 and np.abs(x[1:]).max() < 127
    return x, q


def main() -> None:
    g = np.random.default_rng(0x60_1D)
    # quantisation KATs (A4)
    for name, x in (("rounding_kat", rounding_kat()), ("max_abs_kat", max_abs_kat())):
        q, s = np_ref.quantize_symmetric(x[None])
        np.savez_compressed(HERE / f"{name}.npz", x=x, q=q[0], scale=s)
    # int8 GEMM KATs (A5) with rescale (A6): (f32(c) * a_scale) * w_scale
    arrays = {}
    for name, (a, w) in gemm_patterns().items():
        c = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
        a_s = (g.random(a.shape[0], dtype=np.float32) + np.float32(0.01)) / np.float32(127)
        w_s = (g.random(w.shape[0], dtype=np.float32) + np.float32(0.01)) / np.float32(127)
        outf = (c.astype(np.float32) * a_s[:, None]).astype(np.float32) * w_s[None, :]
        arrays.update({f"{name}_a": a, f"{name}_w": w, f"{name}_c": c, f"{name}_as": a_s, f"{name}_ws": w_s,
                       f"{name}_out": outf.astype(np.float32)})
    mt = gemm_patterns()["mtile_uniform"][0]
    assert np.array_equal(arrays["mtile_uniform_c"],
                          np.repeat((2048 * (np.arange(mt.shape[0]) % 5 + 1)).astype(np.int32)[:, None], 64, axis=1))
    np.savez_compressed(HERE / "gemm_kats.npz", **arrays)
    # weight repack (A1/A2): dequantise, then per-row symmetric int8
    for kind in (4, 6):
        n, k = 24, 768
        blocks = synth.kquant(kind, n, k, index=900 + kind)
        w8, ws = np_ref.quantize_symmetric(np_ref.dequant(kind, blocks, n, k))
        np.savez_compressed(HERE / f"repack_q{kind}k.npz", blocks=blocks, k=k, n=n, w8=w8, scales=ws)
    # Q5_K high bits (A3): single-bit blocks, expected values from the closed form
    blocks, y = q5_k_single_bit_blocks()
    w8, ws = np_ref.quantize_symmetric(y)
    np.savez_compressed(HERE / "repack_q5k_bits.npz", blocks=blocks, k=256, n=y.shape[0], y=y, w8=w8, scales=ws)
    # Q8_K half-to-even ties, in a row of two blocks (the second is N(0,1) data)
    x, q = q8_k_tie_block()
    row = np.concatenate([x, synth.activations(1, 256, index=915)[0]])
    bs = q.reshape(16, 16).sum(axis=1)
    tie_block = np_ref.pack_q8_k(np.array([1.0], np.float32), q[None], bs[None])
    np.savez_compressed(HERE / "q8_k_ties.npz", x=row[None], q8k_block0=tie_block)
    # per-token A8 quantisation with K padded to a multiple of 64
    a = synth.activations(5, 1000, index=910)
    q, s = np_ref.quantize_symmetric(a)
    q_pad = np.zeros((5, 1024), np.int8)
    q_pad[:, :1000] = q
    np.savez_compressed(HERE / "quantize_a8.npz", a=a, k_pad=1024, a8=q_pad, scales=s)
    # Q8_K activations and the decode dots (A9): exact per-block integer sums
    x = synth.activations(3, 1024, index=920)
    x[1, :256] = 0.0  # an all-zero block: d = 0, quants 0
    q8 = np.stack([np_ref.pack_q8_k(*np_ref.quantize_q8_k(row)) for row in x])
    np.savez_compressed(HERE / "q8_k.npz", x=x, q8k=q8)
    for kind in (4, 6):
        n, k = 40, 1024
        w = synth.kquant(kind, n, k, index=930 + kind)
        isum, msum, y, mag = [], [], [], []
        nb = k // 256
        if kind == 4:
            dw, dminw = (v.reshape(n, nb).astype(np.float64) for v in np_ref.q4_k_ints(w)[:2])
        else:
            dw, dminw = np_ref.q6_k_ints(w)[0].reshape(n, nb).astype(np.float64), np.zeros((n, nb))
        for row in x:
            i_, m_, y_ = np_ref.block_sums(kind, w, n, k, row)
            da = np_ref.quantize_q8_k(row)[0].astype(np.float64)[None, :]
            isum.append(i_)
            msum.append(m_)
            y.append(y_)
            # block-level magnitude: the f32 evaluation of the row sum errs by a
            # small multiple of 2^-24 * nb * mag whatever the summation order
            mag.append((np.abs(dw * da * i_) + np.abs(dminw * da * m_)).sum(axis=1))
        np.savez_compressed(HERE / f"gemv_q{kind}k.npz", w=w, k=k, n=n, x=x, q8k=q8, isum=np.stack(isum),
                            msum=np.stack(msum), y=np.stack(y), mag=np.stack(mag))
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
