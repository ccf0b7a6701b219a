"""GPU parity of the four kernels (launch layer, device pointers) against the
C oracle: int8 weights/activations, scales and int32 accumulators bit-exact,
f32 GEMM outputs bit-exact (same operation order), decode GEMV f32 within
1e-5 of the summed block-term magnitude (integer block sums bit-exact)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rocknpu_amd import hip, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# ---------------------------------------------------------------- kernel (a)
@pytest.mark.parametrize("kind,n,k", [
    (4, 1, 256), (4, 67, 2048), (4, 130, 5632), (4, 5632, 2048),
    (5, 48, 2048), (5, 9, 768),
    (6, 1, 256), (6, 33, 2048), (6, 70, 5632), (6, 2048, 5632),
    # one-chunk rows streamed by waves that walk several rows each (more rows than waves)
    (6, 7001, 2048), (4, 13003, 1024), (5, 6500, 512),
])
def test_repack_w8_bit_exact(kind, n, k):
    print(f"repack kind={kind} n={n} k={k}", flush=True)
    blocks = synth.kquant(kind, n, k, index=100 + kind * 7 + n)
    w8_ref, sc_ref = orc.repack_w8(kind, blocks, k, n)
    w8, sc = hip.repack_w8(kind, _dev(blocks), k, n)
    torch.cuda.synchronize()
    w8, sc = w8.cpu().numpy(), sc.cpu().numpy()
    assert np.array_equal(w8[:, :k], w8_ref)
    assert not w8[:, k:].any()
    assert np.array_equal(_bits(sc), _bits(sc_ref))


def test_repack_zero_and_nonfinite_rows():
    k, n = 512, 3
    blocks = synth.q4_k(n, k, index=7).reshape(n, -1, 144).copy()
    blocks[0] = 0                      # all-zero row -> scale 1.0, zero int8
    blocks[2, 1, 0:2] = [0x00, 0x7C]   # d = +inf in one block -> row rejected
    flat = blocks.reshape(-1)
    w8, sc = hip.repack_w8(4, _dev(flat), k, n)
    torch.cuda.synchronize()
    w8, sc = w8.cpu().numpy(), sc.cpu().numpy()
    assert sc[0] == 1.0 and not w8[0].any()
    assert np.isnan(sc[2])
    w8_ref, sc_ref = orc.repack_w8(4, np.ascontiguousarray(blocks[:2].reshape(-1)), k, 2)
    assert np.array_equal(w8[:2, :k], w8_ref) and np.array_equal(_bits(sc[:2]), _bits(sc_ref))


@pytest.mark.parametrize("kind,n,k", [(4, 96, 2048), (4, 40, 4096), (5, 33, 2048), (6, 96, 2048), (6, 20, 5632)])
def test_repack_exact_ties(kind, n, k):
    """Rows whose scale is a power of two, so that many values sit exactly on
    half-integers after scaling: every lane holding one takes the exact
    division and rounds half away from zero, bit for bit with the oracle."""
    print(f"repack ties kind={kind} n={n} k={k}", flush=True)
    from . import np_ref

    blocks = np_ref.tie_rows(kind, n, k, seed=300 + kind + n)
    w8_ref, sc_ref = orc.repack_w8(kind, blocks, k, n)
    w8, sc = hip.repack_w8(kind, _dev(blocks), k, n)
    torch.cuda.synchronize()
    assert np.array_equal(w8.cpu().numpy()[:, :k], w8_ref)
    assert np.array_equal(_bits(sc.cpu().numpy()), _bits(sc_ref))


# ---------------------------------------------------------------- kernel (b)
def _rounding_kat_row() -> np.ndarray:
    """The reference's rounding edge values plus its 2051 LCG values
    (crates/rocknpu-capi/src/lib.rs:5680-5700)."""
    vals = [-12.75, -7.5, -3.5, -1.5, -0.5, -0.49999997, 0.0, 0.49999997, 0.5, 1.5, 3.5, 7.5, 12.75]
    state = 0x12345678
    for _ in range(2051):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        unit = np.float32(state >> 8) / np.float32((1 << 24) - 1)
        vals.append((unit * np.float32(2.0) - np.float32(1.0)) * np.float32(17.0))
    return np.array(vals, np.float32)


# The register kernel sizes its workgroup to the row: one float4 a thread for
# at most 512 rows of at most 4096 values, else two, up to 1024 threads, so
# rows of 2049-3072 float4 take three a thread and longer ones four.
@pytest.mark.parametrize("m,k,k_pad", [(1, 2048, 2048), (128, 2048, 2048), (7, 5632, 5632), (3, 300, 320),
                                       (5, 1001, 1024), (2, 2064, 2112),
                                       (600, 2048, 2048),    # over 512 rows: two float4 a thread
                                       (1, 64, 64), (2, 4, 64),  # one wave
                                       (3, 11264, 11264),    # three float4 a thread
                                       (4, 14336, 14336),    # four float4 a thread, 1024 threads
                                       (2, 16384, 16384),    # the longest row kept in registers
                                       (3, 16388, 16448)])   # longer: two passes over the row
def test_quantize_a8_bit_exact(m, k, k_pad):
    print(f"a8 m={m} k={k} k_pad={k_pad}", flush=True)
    a = synth.activations(m, k, index=200 + m + k)
    a8_ref, sc_ref = orc.quantize_a8(a, k_pad)
    a8, sc = hip.quantize_a8(_dev(a), k_pad)
    torch.cuda.synchronize()
    assert np.array_equal(a8.cpu().numpy(), a8_ref)
    assert np.array_equal(_bits(sc.cpu().numpy()), _bits(sc_ref))


# scalar path; row in registers at one to four float4 a thread; two vector passes
@pytest.mark.parametrize("k", [2051, 2048, 5632, 11264, 14336, 16388])
def test_quantize_a8_edge_rows(k):
    print(f"a8 edge rows k={k}", flush=True)
    kat = np.resize(_rounding_kat_row(), k)
    rows = np.zeros((6, k), np.float32)
    rows[0] = kat
    rows[1] = 0.0                                   # zero row: scale 1.0
    rows[2] = kat * np.float32(1e-38)               # subnormal-range values
    rows[3] = np.float32(127.0) * np.sign(kat)      # scale exactly 1: ties at +-0.5 not hit
    # max 127 gives scale exactly 1.0, so x/scale hits exact ties at +-(j + 0.5)
    ties = np.arange(-126.5, 127.0, 1.0, dtype=np.float32)
    rows[4, 0] = 127.0
    rows[4, 1:1 + ties.size] = ties
    rows[5] = kat
    rows[5, 100] = np.nan
    a8, sc = hip.quantize_a8(_dev(rows), k)
    torch.cuda.synchronize()
    a8, sc = a8.cpu().numpy(), sc.cpu().numpy()
    ref8, refs = orc.quantize_a8(rows[:5], k)
    assert np.array_equal(a8[:5], ref8)
    assert np.array_equal(_bits(sc[:5]), _bits(refs))
    assert sc[1] == 1.0
    assert np.isnan(sc[5]) and not a8[5].any()
    rows[5, 100] = np.inf
    _, sc = hip.quantize_a8(_dev(rows[5:6]), k)
    torch.cuda.synchronize()
    assert np.isnan(sc.cpu().numpy()[0])


# ---------------------------------------------------------------- kernel (c)
def _gemm_dev(a8, as_, w8, ws):
    out_i32 = torch.empty((a8.shape[0], w8.shape[0]), dtype=torch.int32, device=DEV)
    out = hip.gemm_w8a8(_dev(a8), _dev(as_), _dev(w8), _dev(ws), out_i32=out_i32)
    torch.cuda.synchronize()
    return out.cpu().numpy(), out_i32.cpu().numpy()


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (4, 96, 256), (16, 256, 2048), (33, 130, 320),
                                   (128, 5632, 2048), (200, 300, 640), (512, 2048, 2048),
                                   (600, 520, 5632), (1, 5632, 2048), (257, 64, 128),
                                   (300, 300, 64),        # one K step: pipeline prologue only
                                   (4096, 4096, 256),     # 256x256 tiles
                                   (4100, 4000, 192),     # 256x256 tiles, ragged edges, 3 K steps
                                   (64, 48, 192),         # 64x32 tiles, half a tile of N past the edge
                                   (250, 70, 4160),       # 64x32 tiles, K not a multiple of 128: 64-byte stages
                                   (40, 33, 64),          # 64x32 tiles, one K step
                                   (3, 28672, 4096),      # weight-streaming kernel, many tiles per workgroup
                                   (16, 17, 7168),        # weight-streaming kernel at its LDS limit, ragged tile
                                   (9, 100, 64),          # weight-streaming kernel, fewer K chunks than waves
                                   (16, 40, 7232),        # A8 rows beyond the weight-streaming LDS: direct-load tiles
                                   (24, 5632, 2048),      # 17..32 rows: direct-load 64x32 tiles
                                   # 128-byte stages; two stages where tiles outnumber the 256 CUs
                                   (64, 1000, 2048),      # 64x32 tiles, four stages
                                   (64, 16500, 128),      # 64x32 tiles, two stages
                                   (100, 16500, 128),     # 64x64 tiles, two stages, ragged M
                                   (250, 16500, 128),     # 128x64 tiles, two stages, ragged N
                                   (600, 11000, 128),     # 128x128 tiles, two per CU, ragged edges
                                   (520, 16500, 128),     # 256x256 tiles: one round instead of two of 128x128
                                   # larger tiles that fit on the CUs in one round
                                   (64, 8224, 256),       # 64x64 tiles, four stages
                                   (100, 8256, 384),      # 128x64 tiles, four stages, ragged M
                                   (250, 8260, 256),      # 128x128 tiles, three stages, ragged N
                                   (520, 8300, 384),      # 256x128 tiles, eight waves, three stages, ragged edges
                                   (250, 8260, 320),      # 128x128 tiles, K % 128 != 0: 64-byte stages
                                   (520, 8300, 320),      # 256x128 tiles, K % 128 != 0: 64-byte stages
                                   (2040, 11200, 128),    # 3 rounds of 256x128 tiles beat 2 of 256x256
                                   # the smallest of 64x32, 64x64 and 128x64 tiles that fits on the CUs in one round
                                   (120, 1000, 2048),     # 65..128 rows: 64x32 tiles
                                   (200, 2000, 320),      # 64x32 tiles, K % 128 != 0: 64-byte stages
                                   (300, 2000, 384),      # 64x64 tiles
                                   (520, 2050, 128),      # 128x64 tiles
                                   (1000, 2600, 256),     # 128x128 tiles, three stages (128x64 would need two per CU)
                                   (4100, 4000, 256)])    # 256x256 tiles, two stages, ragged edges
def test_gemm_w8a8_bit_exact(m, n, k):
    print(f"gemm m={m} n={n} k={k}", flush=True)
    g = np.random.default_rng(m * 1000 + n + k)
    a8 = g.integers(-127, 128, (m, k), dtype=np.int8)
    w8 = g.integers(-127, 128, (n, k), dtype=np.int8)
    as_ = (g.random(m, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    ws = (g.random(n, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    out, c = _gemm_dev(a8, as_, w8, ws)
    c_ref = orc.gemm_i32(a8, w8, threads=8)
    assert np.array_equal(c, c_ref)
    assert np.array_equal(_bits(out), _bits(orc.rescale(c_ref, as_, ws)))


def test_gemm_reference_kats():
    """Closed-form patterns of the reference's hardware gates."""
    # uniform M-tile: input row%5+1, weights 1 -> K*(row%5+1) (int8_mtile.rs:28-37,71-82)
    m, n, k = 128, 256, 2048
    a8 = np.repeat((np.arange(m) % 5 + 1).astype(np.int8)[:, None], k, axis=1)
    w8 = np.ones((n, k), np.int8)
    _, c = _gemm_dev(a8, np.ones(m, np.float32), w8, np.ones(n, np.float32))
    assert np.array_equal(c, np.repeat((k * (np.arange(m) % 5 + 1))[:, None], n, axis=1))
    # M=1 pattern a=((i*7+3)%9)-4, b=((i*5+1)%11)-5 over N*K (int8_decode_m1.rs:35-45),
    # its negation and a zero input (int8_projection_profile.rs:11-22,54-56)
    k, n = 2048, 96
    a = (((np.arange(k) * 7 + 3) % 9) - 4).astype(np.int8)
    b = (((np.arange(n * k) * 5 + 1) % 11) - 5).astype(np.int8).reshape(n, k)
    ref = b.astype(np.int64) @ a.astype(np.int64)
    for sign in (1, -1, 0):
        _, c = _gemm_dev((a * sign).astype(np.int8)[None, :], np.ones(1, np.float32), b, np.ones(n, np.float32))
        assert np.array_equal(c[0], (ref * sign).astype(np.int32))
    # K-split pattern ((row*7+kk*3+5)%13)-6 / ((col*5+kk*11+3)%17)-8 (int8_mtile_ksplit.rs:27-35)
    m, n, k = 16, 64, 6144
    r, kk = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    a8 = (((r * 7 + kk * 3 + 5) % 13) - 6).astype(np.int8)
    cidx, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    w8 = (((cidx * 5 + kk * 11 + 3) % 17) - 8).astype(np.int8)
    _, c = _gemm_dev(a8, np.ones(m, np.float32), w8, np.ones(n, np.float32))
    assert np.array_equal(c, (a8.astype(np.int64) @ w8.astype(np.int64).T).astype(np.int32))
    # extreme magnitudes: |C| = 127^2 * K stays inside int32
    m, n, k = 8, 64, 8192
    a8 = np.full((m, k), -127, np.int8)
    w8 = np.full((n, k), 127, np.int8)
    w8[1::2] = -127
    _, c = _gemm_dev(a8, np.ones(m, np.float32), w8, np.ones(n, np.float32))
    exp = np.where(np.arange(n) % 2 == 0, -127 * 127 * k, 127 * 127 * k).astype(np.int32)
    assert np.array_equal(c, np.broadcast_to(exp, (m, n)))


def test_w8a8_pipeline_q4k_5632x2048_128_tokens():
    """Repack -> A8 quant -> GEMM for the 5632x2048 Q4_K weight and 128 tokens."""
    m, k, n = 128, 2048, 5632
    blocks = synth.q4_k(n, k, index=0)
    a = synth.activations(m, k, index=1)
    w8, ws = hip.repack_w8(4, _dev(blocks), k, n)
    a8, as_ = hip.quantize_a8(_dev(a))
    out = hip.gemm_w8a8(a8, as_, w8, ws)
    torch.cuda.synchronize()
    ref = orc.matmul_q_w8a8(4, blocks, a, n, threads=8)
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(ref))


@pytest.mark.parametrize("kind,m,k,n,lda", [(4, 128, 2048, 5632, 2048), (6, 37, 5632, 300, 5640), (5, 1, 256, 64, 256)])
def test_matmul_w8a8_f32_device_route(kind, m, k, n, lda):
    """rocknpu_hip_matmul_w8a8_f32 (A8 quantisation into a library workspace + GEMM)
    equals the reference W8A8 route bit for bit, including a strided activation
    matrix and a padded K (5632 -> 5632, 256 -> 256 with 64-aligned k_pad)."""
    print(f"matmul_w8a8_f32 kind={kind} m={m} k={k} n={n}", flush=True)
    blocks = synth.kquant(kind, n, k, index=1200 + m)
    a = synth.activations(m, lda, index=1201 + m)
    w8, ws = hip.repack_w8(kind, _dev(blocks), k, n)
    out = hip.matmul_w8a8_f32(_dev(a), w8, ws, k=k)
    torch.cuda.synchronize()
    ref = orc.matmul_q_w8a8(kind, blocks, np.ascontiguousarray(a[:, :k]), n, threads=8)
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(ref))


# ---------------------------------------------------------------- kernel (d)
@pytest.mark.parametrize("m,k", [(1, 256), (1, 2048), (4, 2048), (3, 5632), (8, 2048), (11, 1024)])
def test_quantize_q8_k_bit_exact(m, k):
    x = synth.activations(m, k, index=300 + m + k)
    if m > 2:
        x[1, :256] = 0.0                   # all-zero block
        x[2, 5] = -np.abs(x[2, :256]).max() - 1.0
        x[2, 9] = -x[2, 5]                 # equal magnitudes: the first one wins
    q = hip.quantize_q8_k(_dev(x))
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), orc.quantize_q8_k(x))


def _gemv_check(kind, n, k, m, index):
    w = synth.kquant(kind, n, k, index=index)
    x = synth.activations(m, k, index=index + 1)
    q8 = orc.quantize_q8_k(x)
    nb = k // 256
    isum = torch.empty((m, n, nb), dtype=torch.int32, device=DEV)
    msum = torch.empty((m, n, nb), dtype=torch.int32, device=DEV)
    out = hip.gemv_q8_k(kind, _dev(w), k, n, _dev(q8), isum=isum, msum=msum)
    torch.cuda.synchronize()
    out, isum, msum = out.cpu().numpy(), isum.cpu().numpy(), msum.cpu().numpy()
    ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=8)
    for mi in range(m):
        ris, rms, mag = orc.gemv_block_sums(kind, w, k, n, q8[mi])
        assert np.array_equal(isum[mi], ris), f"isum row {mi}"
        assert np.array_equal(msum[mi], rms), f"msum row {mi}"
        err = np.abs(out[mi].astype(np.float64) - ref[mi])
        assert np.all(err <= 1e-5 * mag), f"row {mi}: max err/mag {np.max(err / mag)}"
        assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"


@pytest.mark.parametrize("kind,n,k,m", [
    (4, 64, 256, 1), (4, 2048, 2048, 1), (4, 256, 2048, 4), (4, 5632, 2048, 1), (4, 300, 5632, 3),
    (6, 64, 256, 1), (6, 2048, 5632, 1), (6, 2048, 5632, 4), (6, 100, 2048, 8), (4, 130, 14336, 2),
])
def test_gemv_q8_k(kind, n, k, m):
    print(f"gemv kind={kind} n={n} k={k} m={m}", flush=True)
    _gemv_check(kind, n, k, m, index=400 + kind + n + m)


@pytest.mark.parametrize("n,k,m", [(16, 256, 2), (40, 1024, 3), (2048, 2048, 4), (130, 5632, 5), (300, 2048, 8),
                                   (17, 14336, 3), (1000, 4096, 7), (33, 256, 6), (8200, 1024, 3), (11264, 2048, 4)])
def test_gemv_q4k_multi_row(n, k, m):
    """Q4_K at 2..8 activation rows without the exact-sums outputs (3..8 rows run on the
    matrix-core kernel) against the oracle: ragged tiles of 16 weight rows, blocks per row
    not a multiple of 8, padded activation rows; rows of one LDS stage with several tiles
    per workgroup at 3..4 rows (8200 x 1024, 11264 x 2048) take the staged kernel."""
    print(f"gemv multi-row n={n} k={k} m={m}", flush=True)
    w = synth.kquant(4, n, k, index=800 + n + m)
    x = synth.activations(m, k, index=801 + k)
    q8 = orc.quantize_q8_k(x)
    out = hip.gemv_q8_k(4, _dev(w), k, n, _dev(q8))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = orc.gemv_q8_k(4, w, k, n, q8, threads=8)
    for mi in range(m):
        _, _, mag = orc.gemv_block_sums(4, w, k, n, q8[mi])
        err = np.abs(got[mi].astype(np.float64) - ref[mi])
        assert np.all(err <= 1e-5 * mag), f"row {mi}: max err/mag {np.max(err / mag)}"
        assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"


@pytest.mark.parametrize("n,k,m", [(16, 256, 5), (40, 1024, 4), (2048, 5632, 6), (130, 5632, 5), (300, 2048, 8),
                                   (17, 14336, 7), (1000, 4096, 7), (64, 28672, 8),
                                   (4096, 2048, 3), (4200, 1024, 4)])
def test_gemv_q6k_multi_row(n, k, m):
    """Q6_K at 3..8 activation rows without the exact-sums outputs against the oracle
    (5..8 rows run on the matrix-core kernel, and 3..4 rows when the weight rows make
    a 16-row tile per CU): ragged tiles, blocks per row not a multiple of 8, odd row
    lengths (2-byte aligned blocks), padded activation rows, and a K whose activation
    rows need two launches (112 KiB of LDS)."""
    print(f"gemv q6k multi-row n={n} k={k} m={m}", flush=True)
    w = synth.kquant(6, n, k, index=820 + n + m)
    x = synth.activations(m, k, index=821 + k)
    q8 = orc.quantize_q8_k(x)
    out = hip.gemv_q8_k(6, _dev(w), k, n, _dev(q8))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = orc.gemv_q8_k(6, w, k, n, q8, threads=8)
    for mi in range(m):
        _, _, mag = orc.gemv_block_sums(6, w, k, n, q8[mi])
        err = np.abs(got[mi].astype(np.float64) - ref[mi])
        assert np.all(err <= 1e-5 * mag), f"row {mi}: max err/mag {np.max(err / mag)}"
        assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"


def test_gemv_m_chunking():
    """m above one launch's 8 rows is split into launches; results unchanged."""
    _gemv_check(4, 96, 2048, 13, index=500)


@pytest.mark.parametrize("kind,ns,k,m", [
    (4, (2048, 256, 256), 2048, 1), (4, (2048, 256, 256), 2048, 4), (4, (5632, 5632), 2048, 1),
    (4, (5632, 5632), 2048, 4), (6, (2048,), 5632, 1), (6, (2048,), 5632, 4), (4, (96, 160, 32, 64), 1024, 8),
    (6, (130, 70), 2048, 3), (4, (40,), 14336, 2), (4, (33,), 256, 11),
    (6, (300000,), 256, 1),  # grid capped: several prefetch rounds per wave
    # Q4_K rows longer than one 8-block stage: LDS-staged weights at 4, 16 and 8 rows,
    # then rows too long for the staged kernel's LDS (the unstaged matrix-core kernel)
    (4, (1000, 3000), 4096, 4), (4, (700,), 3072, 13), (4, (256, 4100), 6144, 8), (4, (256, 4100), 14336, 8),
    # Q6_K on the LDS stream: 57 blocks per row (every other row starts 2 bytes
    # off a 4-byte boundary; the last step of a row is partial), 16 stream waves
    # at 2 rows with a ragged last workgroup, and 4 rows of 64 blocks on a wide
    # weight (a two-slot ring beside the activations)
    (6, (333,), 14592, 1), (6, (4101,), 14592, 2), (6, (4096,), 16384, 4),
    # four members on the lane kernel and the Q6_K stream (the fourth runs as a
    # launch of its own: the kernels take three members' fields as preloaded
    # arguments)
    (4, (2048, 256, 256, 512), 2048, 1), (6, (2048, 100, 300, 48), 5632, 1),
    # raw rows on the matrix cores beyond 0xffff tiles (runs of 0xffff tiles)
    (4, (65537 * 16 + 5,), 256, 4),
])
def test_gemv_fused_grouped(kind, ns, k, m):
    """Fused Q8_K quant + grouped GEMV == separate quant + per-member GEMV, bit for bit,
    and within tolerance of the oracle."""
    print(f"fused gemv kind={kind} ns={ns} k={k} m={m}", flush=True)
    ws = [synth.kquant(kind, n, k, index=600 + i + n) for i, n in enumerate(ns)]
    x = synth.activations(m, k, index=700 + m + k)
    dx = _dev(x)
    outs = hip.gemv_q_f32(kind, [_dev(w) for w in ws], k, ns, dx)
    q8 = hip.quantize_q8_k(dx)
    torch.cuda.synchronize()
    q8_ref = orc.quantize_q8_k(x)
    assert np.array_equal(q8.cpu().numpy(), q8_ref)
    for w, n, o in zip(ws, ns, outs):
        sep = hip.gemv_q8_k(kind, _dev(w), k, n, q8)
        torch.cuda.synchronize()
        got = o.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), sep.cpu().numpy().view(np.uint32))
        ref = orc.gemv_q8_k(kind, w, k, n, q8_ref, threads=8)
        for mi in range(m):
            _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8_ref[mi])
            err = np.abs(got[mi].astype(np.float64) - ref[mi])
            assert np.all(err <= 1e-5 * mag)
            assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"


@pytest.mark.parametrize("m", [1, 4])
def test_gemv_q6_stream_stall(m):
    """The Q6_K stream kernel's waves wait for the activations with a bounded
    poll. Forced from the host to give up (test hook: one arrival more than the
    workgroup has, 8 polls; every wave still exits), fused and Q8_K-input
    launches write NaN and set the stall flag; with the hook off they match
    each other bit for bit and the oracle, and leave the flag clear."""
    import ctypes

    from rocknpu_amd import _lib

    kind, n, k = 6, 2048, 2048
    mf, lanes, waves = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    arr = (ctypes.c_size_t * 1)(n)
    assert _lib.load().rocknpu_hip_gemv_shape(kind, m, k, arr, 1, 1, 0, ctypes.byref(mf), ctypes.byref(lanes),
                                              ctypes.byref(waves)) == 0
    assert mf.value == 2  # the stream kernel
    w = synth.kquant(kind, n, k, index=2400 + m)
    x = synth.activations(m, k, index=2410 + m)
    dw, dx = _dev(w), _dev(x)
    q8 = hip.quantize_q8_k(dx)
    torch.cuda.synchronize()
    assert not hip.gemv_take_stall()
    print(f"q6 stream stall hook on m={m}", flush=True)
    hip.gemv_test_stall(8)
    try:
        fused = hip.gemv_q_f32(kind, [dw], k, [n], dx)[0]
        torch.cuda.synchronize()
        assert np.isnan(fused.cpu().numpy()).all()
        assert hip.gemv_take_stall()
        sep = hip.gemv_q8_k(kind, dw, k, n, q8)
        torch.cuda.synchronize()
        assert np.isnan(sep.cpu().numpy()).all()
        assert hip.gemv_take_stall()
    finally:
        hip.gemv_test_stall(0)
    print(f"q6 stream stall hook off m={m}", flush=True)
    fused = hip.gemv_q_f32(kind, [dw], k, [n], dx)[0]
    sep = hip.gemv_q8_k(kind, dw, k, n, q8)
    torch.cuda.synchronize()
    assert not hip.gemv_take_stall()
    got = fused.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), sep.cpu().numpy().view(np.uint32))
    q8_ref = orc.quantize_q8_k(x)
    ref = orc.gemv_q8_k(kind, w, k, n, q8_ref, threads=8)
    for mi in range(m):
        _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8_ref[mi])
        err = np.abs(got[mi].astype(np.float64) - ref[mi])
        assert np.all(err <= 1e-5 * mag)
        assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"
