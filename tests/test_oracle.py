"""Pins the C oracle (CPU only): against the reference's own known-answer
tests, an independent numpy restatement (tests/np_ref.py), closed forms and
brute force, with planted mistakes showing each check has teeth."""
import numpy as np
import pytest

from oracle import oracle as orc
from rocknpu_amd import synth

from . import np_ref


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# ------------------------------------------------------------------ formats
def test_block_sizes_match_ggml_abi():
    # crates/rocknpu-capi/src/lib.rs:5729-5736 pins Q4_K = 144 and Q6_K = 210
    assert orc.BLOCK_BYTES[4] == 144 and orc.BLOCK_BYTES[6] == 210
    assert orc.BLOCK_BYTES[5] == 176 and orc.Q8K_BYTES == 292


def test_fp16_exhaustive():
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.fp16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(_bits(got[finite]), _bits(ref[finite]))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_scale_packing_roundtrip():
    g = np.random.default_rng(1)
    sc, mn = g.integers(0, 64, (500, 8)), g.integers(0, 64, (500, 8))
    s2, m2 = np_ref.unpack_k4_scales(synth.pack_scales_k4(sc, mn))
    assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("kind", [4, 5, 6])
def test_dequant_matches_numpy_restatement(kind):
    n, k = 37, 2048
    blocks = synth.kquant(kind, n, k, index=kind)
    assert np.array_equal(_bits(orc.dequant_rows(kind, blocks, k, n)), _bits(np_ref.dequant(kind, blocks, n, k)))


def _q4_block(d=1.0, dmin=0.0, sc=None, mn=None, qs=None):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    sc = np.ones(8, int) if sc is None else np.asarray(sc)
    mn = np.zeros(8, int) if mn is None else np.asarray(mn)
    b[4:16] = synth.pack_scales_k4(sc[None], mn[None])[0]
    b[16:] = np.arange(128, dtype=np.uint8) if qs is None else qs
    return b


def test_dequant_q4_k_closed_forms():
    # d = 1, dmin = 0, unit scales: y equals the 4-bit quant in ggml value order
    b = _q4_block()
    y = orc.dequant_rows(4, b, 256, 1)[0]
    qs = np.arange(128, dtype=np.int32).reshape(4, 32)
    expect = np.concatenate([np.concatenate([qs[j] & 15, qs[j] >> 4]) for j in range(4)]).astype(np.float32)
    assert np.array_equal(y, expect)
    # one sub-block carries scale/min values with bits 4-5 set (the j >= 4 packing path)
    for j in range(8):
        sc = np.zeros(8, int)
        mn = np.zeros(8, int)
        sc[j], mn[j] = 53, 46
        b = _q4_block(d=0.5, dmin=0.25, sc=sc, mn=mn, qs=np.full(128, 0x37, np.uint8))
        y = orc.dequant_rows(4, b, 256, 1)[0]
        q = 7 if j % 2 == 0 else 3
        expect = np.full(256, -0.0, np.float32)
        for s in range(8):
            expect[32 * s:32 * s + 32] = 0.5 * (53 if s == j else 0) * q - 0.25 * (46 if s == j else 0)
        assert np.array_equal(y, expect), f"sub-block {j}"


def test_dequant_q6_k_closed_form():
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([1.0], np.float16).view(np.uint8)
    b[192:208] = 1
    b[0:128] = 0x21  # low nibble 1, high nibble 2
    b[128:192] = 0b11100100  # quarter q gets high bits q
    y = orc.dequant_rows(6, b, 256, 1)[0]
    for p in range(256):
        quarter = (p % 128) // 32
        low = 1 if quarter < 2 else 2
        assert y[p] == (low | (quarter << 4)) - 32, p


def test_planted_dequant_mistake_is_caught():
    """Dropping the `- dmin*m` term or swapping nibble order changes the result."""
    blocks = synth.q4_k(4, 512, index=9)
    good = orc.dequant_rows(4, blocks, 512, 4)
    d, dmin, sc, mn, q = np_ref.q4_k_ints(blocks)
    sub = np.arange(256) // 32
    no_min = ((d[:, None] * sc[:, sub]) * q).astype(np.float32).reshape(4, 512)
    assert not np.array_equal(_bits(good), _bits(no_min))
    swapped = q.reshape(-1, 4, 2, 32)[:, :, ::-1].reshape(-1, 256)
    bad = ((d[:, None] * sc[:, sub]) * swapped - dmin[:, None] * mn[:, sub]).astype(np.float32).reshape(4, 512)
    assert not np.array_equal(_bits(good), _bits(bad))


# ------------------------------------------------------------------ symmetric quant
def _rounding_kat():
    vals = [-12.75, -7.5, -3.5, -1.5, -0.5, -0.49999997, 0.0, 0.49999997, 0.5, 1.5, 3.5, 7.5, 12.75]
    state = 0x12345678
    for _ in range(2051):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        unit = np.float32(state >> 8) / np.float32((1 << 24) - 1)
        vals.append((unit * np.float32(2.0) - np.float32(1.0)) * np.float32(17.0))
    return np.array(vals, np.float32)


def test_quantize_symmetric_reference_rounding_kat():
    # crates/rocknpu-capi/src/lib.rs:5680-5709: edge values plus 2051 LCG values
    x = _rounding_kat()
    q, s = orc.quantize_symmetric_row(x)
    qn, sn = np_ref.quantize_symmetric(x[None])
    assert s == sn[0] and np.array_equal(q, qn[0])
    assert s == np.float32(17.0) / np.float32(127.0) or s == np.abs(x).max() / np.float32(127.0)


def test_quantize_symmetric_exact_ties():
    x = np.concatenate([[127.0], np.arange(-126.5, 127.0, 1.0)]).astype(np.float32)
    q, s = orc.quantize_symmetric_row(x)
    assert s == 1.0
    expect = np.concatenate([[127], np.sign(x[1:]) * (np.floor(np.abs(x[1:])) + 1)]).astype(np.int8)
    assert np.array_equal(q, expect)  # half away from zero, never to even
    # a planted floor(x + 0.5) rounding (the sidecar script's form) differs on negative ties
    assert not np.array_equal(np.floor(x + 0.5).astype(np.int8), expect)


def test_quantize_symmetric_max_abs_and_nonfinite():
    # lib.rs:5714-5726: max-abs KAT, then inf / NaN rejection
    x = ((np.arange(2051) * 7919 % 65521).astype(np.float32) - np.float32(32760.0)) * np.float32(0.001)
    q, s = orc.quantize_symmetric_row(x)
    assert s == np.abs(x).max() / np.float32(127.0)
    for bad in (np.inf, -np.inf, np.nan):
        y = x.copy()
        y[1024] = bad
        with pytest.raises(orc.OracleError):
            orc.quantize_symmetric_row(y)
    q, s = orc.quantize_symmetric_row(np.zeros(64, np.float32))
    assert s == 1.0 and not q.any()


def test_quantize_a8_matches_numpy_and_pads():
    a = synth.activations(9, 1000, index=3)
    a8, sc = orc.quantize_a8(a, 1024)
    qn, sn = np_ref.quantize_symmetric(a)
    assert np.array_equal(a8[:, :1000], qn) and not a8[:, 1000:].any()
    assert np.array_equal(_bits(sc), _bits(sn))


@pytest.mark.parametrize("kind", [4, 5, 6])
def test_repack_matches_numpy(kind):
    n, k = 29, 1024
    blocks = synth.kquant(kind, n, k, index=20 + kind)
    w8, sc = orc.repack_w8(kind, blocks, k, n)
    qn, sn = np_ref.quantize_symmetric(np_ref.dequant(kind, blocks, n, k))
    assert np.array_equal(w8, qn) and np.array_equal(_bits(sc), _bits(sn))


@pytest.mark.parametrize("kind", [4, 5, 6])
def test_repack_exact_ties_round_half_away(kind):
    """Rows whose scale is a power of two put many v / scale exactly on
    half-integers; the oracle rounds them half away from zero as numpy's
    floor-based restatement does, and a planted half-to-even rounding fails."""
    n, k = 6, 512
    blocks = np_ref.tie_rows(kind, n, k, seed=kind)
    vals = np_ref.dequant(kind, blocks, n, k)
    w8, sc = orc.repack_w8(kind, blocks, k, n)
    assert np.all(sc == np.float32(0.5 if kind != 6 else 32.0))
    r = vals / sc[:, None]
    ties = (r - np.floor(r)) == 0.5
    even_differs = ties & (np.rint(r) != np_ref.round_half_away(r))
    assert even_differs.sum() > 20, "the rows must hold ties where the two roundings differ"
    qn, sn = np_ref.quantize_symmetric(vals)
    assert np.array_equal(w8, qn) and np.array_equal(_bits(sc), _bits(sn))
    assert not np.array_equal(w8, np.clip(np.rint(r), -127, 127).astype(np.int8))


def test_repack_rejects_bad_sizes():
    blocks = synth.q4_k(2, 512, index=1)
    with pytest.raises(orc.OracleError):
        orc.repack_w8(4, blocks[:-1], 512, 2)


# ------------------------------------------------------------------ int GEMM + rescale
def test_gemm_i32_brute_force_and_rescale():
    g = np.random.default_rng(5)
    a8 = g.integers(-127, 128, (13, 320), dtype=np.int8)
    w8 = g.integers(-127, 128, (21, 320), dtype=np.int8)
    c = orc.gemm_i32(a8, w8)
    assert np.array_equal(c, (a8.astype(np.int64) @ w8.astype(np.int64).T).astype(np.int32))
    assert np.array_equal(c, orc.gemm_i32(a8, w8, threads=4))
    as_ = g.random(13, dtype=np.float32)
    ws = g.random(21, dtype=np.float32)
    out = orc.rescale(c, as_, ws)
    expect = (c.astype(np.float32) * as_[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(_bits(out), _bits(expect))
    # the other association order (acc*w)*a is a different rounding in general
    other = (c.astype(np.float32) * ws[None, :]).astype(np.float32) * as_[:, None]
    assert not np.array_equal(_bits(out), _bits(other))


def test_matmul_w8a8_route_composition():
    m, k, n = 6, 512, 40
    blocks = synth.q6_k(n, k, index=30)
    a = synth.activations(m, k, index=31)
    out = orc.matmul_q_w8a8(6, blocks, a, n)
    wq, ws = np_ref.quantize_symmetric(np_ref.dequant(6, blocks, n, k))
    aq, as_ = np_ref.quantize_symmetric(a)
    c = (aq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.int32)
    expect = (c.astype(np.float32) * as_[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(_bits(out), _bits(expect))
    bad = a.copy()
    bad[2, 7] = np.nan
    with pytest.raises(orc.OracleError):
        orc.matmul_q_w8a8(6, blocks, bad, n)


def test_hilo_stack_and_sum():
    """Two-part encoding (lib.rs:2045-2082) against numpy: rows kept, residual
    x - f32(q) * scale per row; rows on the int8 grid leave a zero residual; the
    reconstruction q*scale + residual is x wherever the subtraction is exact
    (Sterbenz: residual and dequantised value within a factor 2)."""
    m, k = 5, 700
    a = synth.activations(m, k, index=40)
    grid = (np.arange(k) % 255 - 127).astype(np.float32) * np.float32(0.03125)  # exact multiples of max/127
    grid[0] = np.float32(127 * 0.03125)
    a[3] = grid
    st = orc.hilo_stack(a)
    assert st.shape == (2 * m, k)
    assert np.array_equal(_bits(st[:m]), _bits(a))
    q, s = np_ref.quantize_symmetric(a)
    resid = a - (q.astype(np.float32) * s[:, None]).astype(np.float32)
    assert np.array_equal(_bits(st[m:]), _bits(resid.astype(np.float32)))
    assert not st[m + 3].any()
    # sum of halves
    halves = synth.activations(2 * m, 33, index=41)
    assert np.array_equal(_bits(orc.hilo_sum(halves)), _bits(halves[:m] + halves[m:]))
    bad = a.copy()
    bad[1, 2] = np.inf
    with pytest.raises(orc.OracleError):
        orc.hilo_stack(bad)


def test_hilo_reduces_w8a8_error():
    """The point of the encoding: against the exact f64 product of the dequantised
    weights and the f32 activations, the two-part result is closer than plain W8A8."""
    m, k, n = 8, 1024, 64
    blocks = synth.q4_k(n, k, index=42)
    a = synth.activations(m, k, index=43)
    wq, ws = np_ref.quantize_symmetric(np_ref.dequant(4, blocks, n, k))
    exact = a.astype(np.float64) @ (wq.astype(np.float64) * ws[:, None].astype(np.float64)).T
    plain = orc.matmul_q_w8a8(4, blocks, a, n)
    hilo = orc.matmul_q_hilo(4, blocks, a, n)
    assert np.abs(hilo - exact).max() < 0.1 * np.abs(plain - exact).max()


# ------------------------------------------------------------------ Q8_K and the decode dots
def test_quantize_q8_k_matches_numpy():
    x = synth.activations(1, 2048, index=40)[0]
    x[256:512] = 0.0
    x[600] = -5.0
    x[601] = 5.0  # tie in magnitude: the first one (negative) sets the sign of d
    got = orc.quantize_q8_k(x)[0]
    d, qs, bs = np_ref.quantize_q8_k(x)
    assert np.array_equal(got, np_ref.pack_q8_k(d, qs, bs))
    blk = got[292 * 2:292 * 3]
    # x[600] = -5 comes first, so max = -5, iscale = +25.4, d > 0 and q = -127 / +127
    assert blk[4 + 600 - 512:4 + 602 - 512].view(np.int8).tolist() == [-127, 127]
    assert np.frombuffer(blk[0:4].tobytes(), np.float32)[0] > 0


@pytest.mark.parametrize("kind,k", [(4, 2048), (6, 2048), (4, 5632), (6, 5632)])
def test_vec_dot_block_sums_and_value(kind, k):
    n = 24
    w = synth.kquant(kind, n, k, index=50 + kind)
    x = synth.activations(1, k, index=60)[0]
    q8 = orc.quantize_q8_k(x)
    isum, msum, mag = orc.gemv_block_sums(kind, w, k, n, q8[0])
    ni, nm, y64 = np_ref.block_sums(kind, w, n, k, x)
    assert np.array_equal(isum, ni) and np.array_equal(msum, nm)
    y = orc.gemv_q8_k(kind, w, k, n, q8)[0]
    assert np.all(np.abs(y - y64) <= 1e-5 * mag)
    # planted mistake: dropping the mins term moves Q4_K results far outside the bound
    if kind == 4:
        d, dmin, *_ = np_ref.q4_k_ints(w)
        dq = np_ref.quantize_q8_k(x)[0]
        no_min = (d.reshape(n, -1).astype(np.float64) * dq[None] * ni).sum(axis=1)
        assert np.any(np.abs(no_min - y64) > 1e-5 * mag)


# ------------------------------------------------------------------ the reference's aarch64 NEON forms
def test_neon_quantize_matches_scalar_on_the_reference_kat():
    """The reference's own aarch64 test (lib.rs:5679-5710) asserts that the NEON
    second pass (x * f32(1/scale)) gives the scalar (x / scale) bits on its
    rounding KAT; the oracle's NEON form reproduces that assertion."""
    x = _rounding_kat()
    q, s = orc.quantize_symmetric_row(x)
    qn, sn = orc.quantize_symmetric_row(x, neon=True)
    assert s == sn and np.array_equal(q, qn)


def test_neon_quantize_differs_from_scalar_at_rounding_boundaries():
    """In general x * f32(1/s) and x / s round differently when x / s lies
    within an ulp of a half-integer: then the NEON and scalar builds of the
    reference produce int8 values one apart. Searching N(0,1) rows finds such
    values; they are rare and never more than 1 apart."""
    g = np.random.default_rng(11)
    rows = g.standard_normal((400, 4096)).astype(np.float32)
    diffs = 0
    for r in rows:
        q, s = orc.quantize_symmetric_row(r)
        qn, sn = orc.quantize_symmetric_row(r, neon=True)
        assert s == sn
        d = q.astype(np.int32) - qn.astype(np.int32)
        assert np.abs(d).max() <= 1
        diffs += int(np.count_nonzero(d))
    assert 0 < diffs < 1e-4 * rows.size
    # an exact construction: x = 0.5 * s rounds to 1 by division; the reciprocal
    # product lands just below 0.5 when f32(1/s) * s < 1
    for s in np.float32(np.linspace(0.01, 1.0, 5000)):
        inv = np.float32(1.0) / s
        if np.float32(inv * s) < np.float32(1.0):
            x = np.float32(s * np.float32(0.5))
            if x / s == np.float32(0.5) and np.float32(x * inv) < np.float32(0.5):
                row = np.zeros(8, np.float32)
                row[0], row[1] = np.float32(127.0) * s, x
                q, _ = orc.quantize_symmetric_row(row)
                qn, _ = orc.quantize_symmetric_row(row, neon=True)
                if orc.quantize_symmetric_row(row)[1] == s:
                    assert q[1] == 1 and qn[1] == 0
                    break
    else:
        pytest.fail("no boundary case constructed")


def test_neon_rescale_order():
    """rescale_i32_row_neon (lib.rs:664-690) computes (c * w) * a for 4-column
    chunks and the scalar (c * a) * w for the tail; the two orders differ in the
    last bits for some outputs; each order rounds twice (error <= 2^-23
    relative), so they agree to within 2^-22 relative."""
    g = np.random.default_rng(12)
    c = g.integers(-2**24, 2**24, (16, 70), dtype=np.int32)
    a = g.random(16, dtype=np.float32) + np.float32(0.5)
    w = g.random(70, dtype=np.float32) + np.float32(0.5)
    scalar = orc.rescale(c, a, w)
    neon = orc.rescale(c, a, w, neon=True)
    expect = ((c.astype(np.float32) * w[None, :]).astype(np.float32) * a[:, None]).astype(np.float32)
    assert np.array_equal(_bits(neon[:, :68]), _bits(expect[:, :68]))
    assert np.array_equal(_bits(neon[:, 68:]), _bits(scalar[:, 68:]))  # tail of 70 % 4 = 2 columns
    assert not np.array_equal(_bits(neon), _bits(scalar))
    rel = np.abs(neon.astype(np.float64) - scalar) / np.abs(scalar.astype(np.float64))
    assert rel.max() <= 2.0 ** -22
