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


def _split(kind, m, nb):
    """Whether a tiled launch of m rows splits each tile's blocks in ranges
    (rocknpu_hip_gemv_q_f32_tiled): rows of 17-31 blocks at 2-8 rows, of
    32-64 blocks at 1-8 rows."""
    return kind in (4, 6) and ((2 <= m <= 8 and 17 <= nb <= 31) or (1 <= m <= 8 and 32 <= nb <= 64))


def _same_order_as_raw(nb, m=16):
    """Whether the tiled kernels add a row's block terms in the order of the
    raw-row matrix-core kernel (8 waves): rows of at most 16 blocks whatever
    the tiled launch's waves, and rows of 17-31 blocks (8 waves there) where
    the launch does not split."""
    return nb < 32 and not _split(4, m, nb)


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
# register tiles; launches of more than four tiles a CU on eight waves.
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
    (4, 3072, [3072, 100], (3, 4, 9)),        # 12 blocks on 16 waves (4 without a block)
    (6, 2560, [500], (2, 8)),                  # 10 blocks on 16 waves
    (4, 5632, [2048, 300], (2, 3, 5, 8, 12)),  # 22 blocks: split at 2-8 rows, not at 12
    (6, 4352, [40, 2048], (2, 7)),             # 17 blocks: ranges of 9 and 8
    (4, 7936, [33], (4,)),                     # 31 blocks: ranges of 15 and 16
    (6, 8192, [2048], (1, 4)),                 # 32 blocks: 4 ranges of 8 on 8 waves
    (6, 8448, [300, 17], (1, 3, 8)),           # 33 blocks: 4 ranges of 8-9 on 16 waves
    (4, 16384, [64], (2,)),                    # 64 blocks: 4 ranges of 16 on 16 waves
    (4, 512, [100], (1, 3)),
    (6, 256, [40], (1, 2)),
    (4, 2048, [1000, 17], (4, 13)),
    (6, 2048, [32000], (1, 4, 8)),             # 2000 tiles: a workgroup per four (pipelined)
    (4, 2048, [8192, 8192, 2000], (3, 4)),     # 1149 tiles: the same, bits of the raw rows
    (4, 2048, [2048, 256, 256, 512], (1, 4)),  # four members: the fourth a launch of its own
    (6, 5632, [2048, 48, 100, 16], (4,)),      # the same for split launches
    (4, 256, [65537 * 16 + 5], (1,)),          # more than 0xffff tiles: runs of 0xffff tiles
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
        raw_mfma = kind == 4 and 3 <= m <= 16 and nb >= 8 and _same_order_as_raw(nb, m)
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
    miss; one-row calls over rows the one-row rule keeps raw (4 blocks) read
    the raw rows."""
    k, n = 1024, 2048
    assert not hip.gemv_tiled_preferred(4, 1, k) and hip.gemv_tiled_preferred(4, 4, k)
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


def test_split_grouped_equals_separate_and_q8k_input():
    """Split launches (22-block rows at 4 and 6 rows): a member's results are
    the same bits alone, grouped with another member of either size, and from
    Q8_K input; within the oracle bounds."""
    k = 5632
    ws = [synth.kquant(6, n, k, index=3500 + i) for i, n in enumerate((2048, 48))]
    td = [hip.gemv_tile_weights(6, _dev(w), k, n) for w, n in zip(ws, (2048, 48))]
    for m in (4, 6):
        print(f"split grouping m={m}", flush=True)
        x = synth.activations(m, k, index=3510 + m)
        xd = _dev(x)
        both = hip.gemv_q_f32_tiled(6, td, k, [2048, 48], xd)
        alone = [hip.gemv_q_f32_tiled(6, [t], k, [n], xd)[0] for t, n in zip(td, (2048, 48))]
        q8 = hip.quantize_q8_k(xd)
        fromq = [hip.gemv_q8_k_tiled(6, t, k, n, q8) for t, n in zip(td, (2048, 48))]
        torch.cuda.synchronize()
        for i, n in enumerate((2048, 48)):
            got = both[i].cpu().numpy()
            assert np.array_equal(_bits(got), _bits(alone[i].cpu().numpy())), ("grouped vs alone", m, n)
            assert np.array_equal(_bits(got), _bits(fromq[i].cpu().numpy())), ("fused vs Q8_K input", m, n)
            _check_vs_oracle(6, ws[i], k, n, x, got)


def test_split_workspace_left_clear_and_dirty_detected():
    """Every completed split call leaves its workspace zero; a workspace with a
    slot left set always sets the error word (the check clears it), and the
    output there is NaN or, when the other range swaps between the finder's
    swap and its emptying the slot, the exact sum: never other bits. Zeroed
    again, the call is exact."""
    k, n, m = 5632, 2048, 4
    w = synth.kquant(6, n, k, index=3600)
    td = [hip.gemv_tile_weights(6, _dev(w), k, n)]
    xd = _dev(synth.activations(m, k, index=3601))
    nbytes = hip.gemv_tiled_workspace_bytes(6, m, k, n)
    assert nbytes == 256 + (n // 16) * 64 * 8
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    print("split clean calls", flush=True)
    ref = hip.gemv_q_f32_tiled(6, td, k, [n], xd, workspace=ws)[0].cpu().numpy()
    again = hip.gemv_q_f32_tiled(6, td, k, [n], xd, workspace=ws)[0].cpu().numpy()
    assert np.array_equal(_bits(ref), _bits(again))
    assert not ws.any().item()
    assert hip.gemv_workspace_check(ws)
    # a slot left holding a value (tile 3, lane 5, which holds row 53 of
    # activation row 0): the first arrival there finds a tag of no launch
    slots = ws[256:].view(torch.int64)
    slots[3 * 64 + 5] = (1 << 32) | 0x3F800000  # tag 1: no launch's (tags are 2 or more)
    print("split dirty call", flush=True)
    got = hip.gemv_q_f32_tiled(6, td, k, [n], xd, workspace=ws)[0].cpu().numpy()
    assert not hip.gemv_workspace_check(ws)
    at = np.zeros(got.shape, bool)
    at[0, 3 * 16 + 5] = True
    assert np.array_equal(_bits(got[~at]), _bits(ref[~at]))
    assert np.isnan(got[at][0]) or _bits(got[at])[0] == _bits(ref[at])[0]
    ws.zero_()
    fixed = hip.gemv_q_f32_tiled(6, td, k, [n], xd, workspace=ws)[0].cpu().numpy()
    assert np.array_equal(_bits(fixed), _bits(ref)) and hip.gemv_workspace_check(ws)


def test_split_needs_a_workspace():
    import ctypes
    from rocknpu_amd import _lib
    k, n, m = 5632, 32, 4
    t = hip.gemv_tile_weights(6, _dev(synth.kquant(6, n, k, index=3700)), k, n)
    x = _dev(synth.activations(m, k, index=3701))
    out = torch.empty((m, n), device=DEV)
    arr = lambda ty, *v: (ty * len(v))(*v)  # noqa: E731
    st = _lib.load().rocknpu_hip_gemv_q_f32_tiled(6, 1, arr(ctypes.c_void_p, t.data_ptr()), arr(ctypes.c_size_t, t.numel()),
                                                  arr(ctypes.c_size_t, n), k, ctypes.c_void_p(x.data_ptr()), k, m,
                                                  arr(ctypes.c_void_p, out.data_ptr()), arr(ctypes.c_size_t, n),
                                                  None, 0, None)
    assert st == -1
    small = torch.zeros(256, dtype=torch.uint8, device=DEV)
    with pytest.raises(hip.LaunchError):
        hip.gemv_q_f32_tiled(6, [t], k, [n], x, workspace=small)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_split_graph_replays_match_eager():
    """A split launch captured on a stream that already has its workspace (one
    eager call first) replays the eager bits, every replay; capturing on a
    stream without one raises instead of running unsplit."""
    k, ns, m = 5632, [2048], 4
    td = [hip.gemv_tile_weights(6, _dev(synth.kquant(6, ns[0], k, index=3800)), k, ns[0])]
    x = _dev(synth.activations(m, k, index=3801))
    eager = hip.gemv_q_f32_tiled(6, td, k, ns, x)[0].cpu().numpy()
    outs = [torch.empty((m, ns[0]), device=DEV)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hip.gemv_q_f32_tiled(6, td, k, ns, x, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        hip.gemv_q_f32_tiled(6, td, k, ns, x, outs=outs)
    for rep in range(3):
        print(f"split graph replay {rep}", flush=True)
        outs[0].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(outs[0].cpu().numpy()), _bits(eager)), rep
        hip.gemv_q_f32_tiled(6, td, k, ns, x)  # eager work between replays
        torch.cuda.synchronize()
    fresh = torch.cuda.Stream()
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(hip.LaunchError):
        with torch.cuda.graph(g2, stream=fresh):
            hip.gemv_q_f32_tiled(6, td, k, ns, x, outs=outs)
