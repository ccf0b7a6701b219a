"""Decode GEMV on the decode cache's tile-interleaved copies (the launch layer's
rocknpu_hip_gemv_tile_weights / _q_f32_tiled / _q8_k_tiled, and the C ABI's
decode entries from two rows): the copy equals an independent numpy
restatement of the layout byte for byte; the GEMV is within 1e-5 of the
oracle's per-block magnitude and normwise (max|err| / max|y| <= 1e-5); fused
and Q8_K-input calls agree bit for bit, and so do the tiled and raw-row
matrix-core kernels wherever both run with the same waves; graph replays equal
the eager result."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rocknpu_amd import hip, synth
from rocknpu_amd.capi import Context
from tests import np_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bits(x) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _check_vs_oracle(kind, w, k, n, x, got):
    """Per output |err| <= 1e-5 * (sum of block-term magnitudes), and normwise
    max|err| / max|y| <= 1e-5 per activation row."""
    q8 = orc.quantize_q8_k(x)
    ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=8)
    g = got.astype(np.float64)
    for mi in range(x.shape[0]):
        _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[mi])
        err = np.abs(g[mi] - ref[mi])
        assert np.all(err <= 1e-5 * mag), (kind, k, n, mi)
        assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), (kind, k, n, mi)


def _same_order_as_raw(nb):
    """Whether the tiled kernels add a row's block terms in the order of the
    raw-row matrix-core kernel (8 waves): rows of at most 16 blocks whatever
    the tiled launch's waves, and rows of 17-31 blocks (8 waves there)."""
    return nb < 32


@pytest.mark.parametrize("kind,k,n", [
    (4, 2048, 2048), (4, 2048, 333), (4, 4096, 17), (4, 256, 1),
    (6, 5632, 2048), (6, 2048, 1000), (6, 256, 5),
])
def test_tile_weights_equal_the_restatement(kind, k, n):
    print(f"tile weights kind={kind} k={k} n={n}", flush=True)
    w = synth.kquant(kind, n, k, index=3000 + kind + n)
    got = hip.gemv_tile_weights(kind, _dev(w), k, n)
    torch.cuda.synchronize()
    want = np_ref.tile_weights(kind, w, n, k)
    assert got.numel() == want.size == hip.gemv_tiled_bytes(kind, k, n)
    assert np.array_equal(got.cpu().numpy(), want)


# (kind, k, member rows, activation rows): TinyLlama o, qkv, gate+up and down
# (one, one, three and three items per wave), Llama-3-8B q/o and q/k/v (two
# block indices per wave, the second quantised after the first item), gate+up
# (16 waves, seven tiles per workgroup: the item loop) and down (16 waves, four
# blocks per wave; at 5-8 rows the item loop), rows shorter than eight blocks,
# a single block, ragged N; 9-16 activation rows run the item loop on 16-row
# register tiles.
CASES = [
    (4, 2048, [2048], (1, 2, 3, 4, 8, 16)),
    (4, 2048, [2048, 256, 256], (2, 4, 5, 9)),
    (4, 2048, [5632, 5632], (2, 4, 8)),
    (6, 5632, [2048], (1, 2, 4, 6, 8)),
    (4, 4096, [14336, 14336], (1, 4)),
    (4, 4096, [4096], (1, 2, 4, 8)),
    (4, 4096, [4096, 1024, 1024], (3, 6)),
    (6, 4096, [1000], (2, 7)),
    (6, 14336, [4096], (1, 4, 5, 8)),
    (4, 512, [100], (1, 3)),
    (6, 256, [40], (1, 2)),
    (4, 2048, [1000, 17], (4, 13)),
]


@pytest.mark.parametrize("kind,k,ns,ms", CASES)
def test_tiled_gemv(kind, k, ns, ms):
    ws = [synth.kquant(kind, n, k, index=3100 + i + kind * 10 + len(ns)) for i, n in enumerate(ns)]
    wd = [_dev(w) for w in ws]
    td = [hip.gemv_tile_weights(kind, w, k, n) for w, n in zip(wd, ns)]
    nb = k // 256
    for m in ms:
        print(f"tiled gemv kind={kind} k={k} ns={ns} m={m}", flush=True)
        x = synth.activations(m, k, index=3200 + m + k)
        xd = _dev(x)
        fused = hip.gemv_q_f32_tiled(kind, td, k, ns, xd)
        q8 = hip.quantize_q8_k(xd)
        fromq = [hip.gemv_q8_k_tiled(kind, t, k, n, q8) for t, n in zip(td, ns)]
        raw = hip.gemv_q_f32(kind, wd, k, ns, xd)
        torch.cuda.synchronize()
        # the raw rows take the matrix cores from 3 rows (Q4_K); with 8 or more
        # blocks per row both kernels run 8-wave orders
        raw_mfma = kind == 4 and 3 <= m <= 16 and nb >= 8 and _same_order_as_raw(nb)
        for i, n in enumerate(ns):
            got = fused[i].cpu().numpy()
            assert np.array_equal(_bits(got), _bits(fromq[i].cpu().numpy())), "fused vs Q8_K input"
            if raw_mfma:
                assert np.array_equal(_bits(got), _bits(raw[i].cpu().numpy())), "tiled vs raw rows"
            _check_vs_oracle(kind, ws[i], k, n, x, got)


def test_tiled_graph_replays_match_eager():
    kind, k, ns, m = 4, 2048, [5632, 5632], 4
    td = [hip.gemv_tile_weights(kind, _dev(synth.kquant(kind, n, k, index=3300 + i)), k, n) for i, n in enumerate(ns)]
    x = _dev(synth.activations(m, k, index=3301))
    eager = [o.cpu().numpy() for o in hip.gemv_q_f32_tiled(kind, td, k, ns, x)]
    outs = [torch.empty((m, n), device=DEV) for n in ns]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hip.gemv_q_f32_tiled(kind, td, k, ns, x, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hip.gemv_q_f32_tiled(kind, td, k, ns, x, outs=outs)
    for rep in range(3):
        print(f"tiled graph replay {rep}", flush=True)
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert np.array_equal(_bits(o.cpu().numpy()), _bits(e)), rep
        hip.gemv_q_f32_tiled(kind, td[:1], k, ns[:1], x[:1])  # eager work between replays
        torch.cuda.synchronize()


def test_capi_decode_rows_read_the_tiled_copy():
    """The C ABI's decode entries from two rows read the tiled copy it builds
    once per weight: results within the oracle bound, equal to the launch
    layer's tiled call, the copy's bytes counted as resident and its build as a
    miss; one-row calls keep the raw rows."""
    k, n = 2048, 2048
    w4 = synth.q4_k(n, k, index=3400)
    w6 = synth.q6_k(n, k, index=3401)
    x1 = synth.activations(1, k, index=3402)
    x4 = synth.activations(4, k, index=3403)
    with Context() as c:
        out1 = np.empty((1, n), np.float32)
        assert c.matmul_q_q8k(4, w4, x1, out1, k, n) == 0
        s1 = c.decode_cache_stats()
        assert (s1.entries, s1.resident_bytes, s1.misses) == (1, w4.nbytes, 1)
        out4 = np.empty((4, n), np.float32)
        assert c.matmul_q_q8k(4, w4, x4, out4, k, n) == 0
        s2 = c.decode_cache_stats()
        tb = hip.gemv_tiled_bytes(4, k, n)
        assert (s2.entries, s2.resident_bytes, s2.misses, s2.hits) == (1, w4.nbytes + tb, 2, 0)
        assert c.matmul_q_q8k(4, w4, x4, out4, k, n) == 0
        assert c.decode_cache_stats().hits == 1
        _check_vs_oracle(4, w4, k, n, x4, out4)
        want = hip.gemv_q_f32_tiled(4, [hip.gemv_tile_weights(4, _dev(w4), k, n)], k, [n], _dev(x4))[0]
        assert np.array_equal(_bits(out4), _bits(want.cpu().numpy()))
        # the grouped entry, mixed kinds, four rows
        outs = [np.empty((4, n), np.float32) for _ in range(2)]
        assert c.matmul_q_q8k_group([w4, w6], [4, 6], [n, n], x4, outs, k) == 0
        _check_vs_oracle(4, w4, k, n, x4, outs[0])
        _check_vs_oracle(6, w6, k, n, x4, outs[1])
        assert np.array_equal(_bits(outs[0]), _bits(out4))
