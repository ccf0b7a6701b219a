"""K-split W8A8 GEMM on the GPU (rocknpu_hip_gemm_w8a8_ws / _tile): every tile
and split count gives the oracle's int32 accumulators and f32 outputs bit for
bit and leaves the workspace zeroed; routed splits agree through the launch
layer, the device-pointer prompt route and the C ABI; graph replays of split
launches agree with the eager result; the module's workspaces are per stream
and never made under capture; dirty counters are reported, not trusted."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rocknpu_amd import hip, synth
from rocknpu_amd.capi import Context

pytestmark = pytest.mark.gpu
DEV = "cuda"

TILES = [(32, 64, 4), (64, 32, 4), (64, 32, 2), (64, 64, 4), (64, 64, 2), (128, 64, 4), (128, 64, 2),
         (128, 128, 3), (128, 128, 2), (256, 128, 3), (256, 256, 2)]


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _operands(m, n, k, seed):
    g = np.random.default_rng(seed)
    a8 = g.integers(-127, 128, (m, k), dtype=np.int8)
    w8 = g.integers(-127, 128, (n, k), dtype=np.int8)
    as_ = (g.random(m, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    ws = (g.random(n, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    return a8, w8, as_, ws


def _counter_bytes(m, n, bm, bn):
    return 16384, -(-m // bm) * -(-n // bn)


def _eff_splits(k, splits):
    """Splits that get K stages (128 bytes, or 64 when K % 128 != 0): seven
    asked for over 17 stages run as six of three stages."""
    ks = k // 128 if k % 128 == 0 else k // 64
    if splits <= 1 or ks <= 1:
        return 1
    per = -(-ks // splits)
    return -(-ks // per)


def _state_zero(work, m, n, k, bm, bn, splits):
    """The counter block and the stamps of a K-split workspace are all zero (the
    partial tiles between them keep the last call's values)."""
    cb, t = _counter_bytes(m, n, bm, bn)
    units = t * _eff_splits(k, splits)
    stamps = cb + units * bm * bn * 4
    return not work[:cb].any().item() and not work[stamps:stamps + units * 4].any().item()


def _ws_bytes(m, n, bm, bn, splits):
    """Bytes of a K-split workspace: the 16 KiB counter block, the int32
    partial tiles, then one stamp per (tile, split) rounded up to 256 bytes."""
    cb, t = _counter_bytes(m, n, bm, bn)
    units = t * splits
    return cb + units * bm * bn * 4 + -(-units * 4 // 256) * 256


@pytest.mark.parametrize("m,n,k", [
    (128, 512, 2048),   # 16 stages of 128 bytes
    (100, 300, 5632),   # ragged edges, 44 stages
    (37, 200, 1088),    # K % 128 != 0: 17 stages of 64 bytes (seven splits become six)
    (64, 256, 8192),
    (260, 130, 1024),   # 256-row tiles past the edge
])
def test_split_every_tile_bit_exact(m, n, k):
    a8, w8, as_, ws = _operands(m, n, k, m * 7 + n + k)
    c_ref = orc.gemm_i32(a8, w8, threads=8)
    out_ref = _bits(orc.rescale(c_ref, as_, ws))
    d = [torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)]
    for bm, bn, st in TILES:
        cb, t = _counter_bytes(m, n, bm, bn)
        if bm == 32 and k % 128 != 0:
            # 32-row tiles run 128-byte stages only: refused, not run
            with pytest.raises(hip.LaunchError):
                hip.gemm_w8a8_tile(bm, bn, st, 1, d[0], d[1], d[2], d[3])
            continue
        for sp in (1, 2, 3, 4, 7):
            print(f"split gemm m={m} n={n} k={k} tile={bm}x{bn}/{st} splits={sp}", flush=True)
            work = torch.zeros(_ws_bytes(m, n, bm, bn, sp), dtype=torch.uint8, device=DEV) if sp > 1 else None
            c = torch.full((m, n), -1, dtype=torch.int32, device=DEV)
            out = hip.gemm_w8a8_tile(bm, bn, st, sp, d[0], d[1], d[2], d[3], out_i32=c, workspace=work)
            torch.cuda.synchronize()
            assert np.array_equal(c.cpu().numpy(), c_ref), (bm, bn, st, sp)
            assert np.array_equal(_bits(out.cpu().numpy()), out_ref), (bm, bn, st, sp)
            if work is not None:
                assert _state_zero(work, m, n, k, bm, bn, sp), "counters or stamps not left at zero"
                assert hip.gemm_workspace_check(work)


def test_routed_split_through_every_entry():
    """128 x 2048 x 5632 (TinyLlama down at 128 tokens) splits K in two on the
    route: launch layer with and without a workspace, the prompt route and the
    C ABI agree with the oracle; calls of another shape in between."""
    m, k, n = 128, 5632, 2048
    nbytes, splits = hip.gemm_workspace(m, n, k)
    assert splits == 2 and nbytes > 0
    blocks = synth.q6_k(n, k, index=40)
    act = synth.activations(m, k, index=41)
    ref = orc.matmul_q_w8a8(6, blocks, act, n, threads=8)
    w8, wsc = hip.repack_w8(6, torch.from_numpy(blocks).to(DEV), k, n)
    a = torch.from_numpy(act).to(DEV)
    a8, asc = hip.quantize_a8(a)
    work = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    outs = []
    for step in range(3):
        print(f"routed split step {step}", flush=True)
        outs.append(hip.gemm_w8a8(a8, asc, w8, wsc, workspace=work))
        outs.append(hip.gemm_w8a8(a8, asc, w8, wsc, workspace=None))
        outs.append(hip.matmul_w8a8_f32(a, w8, wsc))
        # a smaller split shape in between, on the same workspace
        hip.gemm_w8a8(a8[:32], asc[:32], w8[:1024], wsc[:1024], workspace=work)
    torch.cuda.synchronize()
    assert not work[:16384].any().item() and hip.gemm_workspace_check(work)
    for o in outs:
        assert np.array_equal(_bits(o.cpu().numpy()), _bits(ref))
    with Context() as ctx:
        host = np.empty((m, n), np.float32)
        for _ in range(2):
            assert ctx.matmul_q(6, blocks, act, host, k, n) == 0
            assert np.array_equal(_bits(host), _bits(ref))


def test_split_graph_replays_match_eager():
    m, n, k = 128, 2048, 8192
    assert hip.gemm_workspace(m, n, k)[1] > 1
    a8, w8, as_, ws = _operands(m, n, k, 5)
    d = [torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)]
    eager = hip.gemm_w8a8(*d)
    torch.cuda.synchronize()
    want = _bits(eager.cpu().numpy())
    out = torch.empty_like(eager)
    # the graph's split launches use a workspace of their own, zeroed before capture
    work = torch.zeros(hip.gemm_workspace(m, n, k)[0], dtype=torch.uint8, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hip.gemm_w8a8(*d, out=out, workspace=work)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hip.gemm_w8a8(*d, out=out, workspace=work)
        hip.gemm_w8a8(*d, out=out, workspace=work)
    for rep in range(4):
        print(f"split graph replay {rep}", flush=True)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out.cpu().numpy()), want), rep
        assert not work[:16384].any().item() and hip.gemm_workspace_check(work), rep
        # eager work between replays, on the module's workspace
        hip.gemm_w8a8(d[0][:64], d[1][:64], d[2], d[3])
        torch.cuda.synchronize()


def test_module_workspace_first_made_under_capture_then_eager():
    """A split shape met for the first time under graph capture: the module
    makes no workspace there (the captured call runs unsplit), so the eager
    calls after it, which make and zero one, and the graph's replays all give
    the eager bits."""
    m, n, k = 128, 2048, 5632
    assert hip.gemm_workspace(m, n, k)[1] > 1
    hip._workspaces.clear()
    a8, w8, as_, ws = _operands(m, n, k, 9)
    want = _bits(orc.rescale(orc.gemm_i32(a8, w8, threads=8), as_, ws))
    d = [torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)]
    out_g = torch.empty((m, n), dtype=torch.float32, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hip.gemm_w8a8(*d, out=out_g)
    assert not hip._workspaces, "a workspace was made during capture"
    for rep in range(3):
        print(f"capture-first replay {rep}", flush=True)
        out_g.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out_g.cpu().numpy()), want), rep
        eager = hip.gemm_w8a8(*d)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(eager.cpu().numpy()), want), rep
        assert len(hip._workspaces) == 1
        ws_t = next(iter(hip._workspaces.values()))
        assert not ws_t[:16384].any().item() and hip.gemm_workspace_check(ws_t)


def test_module_workspace_per_stream():
    """Two streams get two workspaces; both give the eager bits, and each is
    left zeroed."""
    m, n, k = 128, 2048, 8192
    hip._workspaces.clear()
    a8, w8, as_, ws = _operands(m, n, k, 11)
    want = _bits(orc.rescale(orc.gemm_i32(a8, w8, threads=8), as_, ws))
    d = [torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for st in streams:
        with torch.cuda.stream(st):
            outs.append(hip.gemm_w8a8(*d))
    torch.cuda.synchronize()
    assert len(hip._workspaces) == 2
    for o in outs:
        assert np.array_equal(_bits(o.cpu().numpy()), want)
    for w in hip._workspaces.values():
        assert not w[:16384].any().item() and hip.gemm_workspace_check(w)


@pytest.mark.parametrize("start", [1, 5])
def test_dirty_workspace_is_reported(start):
    """Counters that are not zero at entry are detected, not trusted. With the
    first tile's counter at 5 (past the split count) every arrival sees it: the
    tile's f32 results are NaN and the error word is set. At 1 (one split
    early) the early last arrival either finds the other split's stamp (its
    partial complete: exact bits) or not (NaN and the flag), so each value of
    the tile is exact or NaN, and any NaN comes with the flag. Wrong bits never.
    The other tiles are exact. After the workspace is zeroed again, a call is
    exact and clean. Every access stays inside the workspace and no wave waits."""
    m, n, k = 128, 512, 8192
    bm, bn, st, sp = 64, 64, 4, 2
    a8, w8, as_, ws = _operands(m, n, k, 21)
    c_ref = orc.gemm_i32(a8, w8, threads=8)
    want = _bits(orc.rescale(c_ref, as_, ws))
    d = [torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)]
    work = torch.zeros(_ws_bytes(m, n, bm, bn, sp), dtype=torch.uint8, device=DEV)
    work.view(torch.int32)[0] = start  # tile 0: rows 0-63, columns 0-63
    out = hip.gemm_w8a8_tile(bm, bn, st, sp, *d, workspace=work)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    tile = got[:64, :64]
    mask = np.ones((m, n), bool)
    mask[:64, :64] = False
    assert np.array_equal(_bits(got)[mask], want[mask])
    clean = hip.gemm_workspace_check(work)
    if start >= sp:
        assert np.isnan(tile).all() and not clean
    else:
        nan = np.isnan(tile)
        assert np.array_equal(_bits(tile)[~nan], want[:64, :64][~nan]), "wrong bits from a dirty counter"
        if nan.any():
            assert not clean
    assert hip.gemm_workspace_check(work), "the check clears the error word"
    work.zero_()
    out = hip.gemm_w8a8_tile(bm, bn, st, sp, *d, workspace=work)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out.cpu().numpy()), want)
    assert hip.gemm_workspace_check(work) and _state_zero(work, m, n, k, bm, bn, sp)


def test_split_extreme_magnitudes_at_the_largest_exact_k():
    """|C| = 127^2 * K at K = 133120, the largest K whose int32 sums are exact
    (127 * 127 * 133120 = 2,147,092,480 < 2^31): the split partials and their sum
    stay exact, on the routed split and on 16 splits."""
    m, n, k = 64, 256, 133120
    nbytes, splits = hip.gemm_workspace(m, n, k)
    assert splits > 1
    a8 = torch.full((m, k), -127, dtype=torch.int8, device=DEV)
    w8 = torch.full((n, k), 127, dtype=torch.int8, device=DEV)
    w8[1::2] = -127
    ones_m = torch.ones(m, device=DEV)
    ones_n = torch.ones(n, device=DEV)
    exp = np.where(np.arange(n) % 2 == 0, -127 * 127 * k, 127 * 127 * k).astype(np.int32)
    exp = np.broadcast_to(exp, (m, n))
    c = torch.empty((m, n), dtype=torch.int32, device=DEV)
    out = hip.gemm_w8a8(a8, ones_m, w8, ones_n, out_i32=c, workspace=torch.zeros(nbytes, dtype=torch.uint8, device=DEV))
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), exp)
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(orc.rescale(exp, np.ones(m, np.float32), np.ones(n, np.float32))))
    work = torch.zeros(_ws_bytes(m, n, 64, 32, 16), dtype=torch.uint8, device=DEV)
    c.fill_(0)
    hip.gemm_w8a8_tile(64, 32, 4, 16, a8, ones_m, w8, ones_n, out_i32=c, workspace=work)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), exp)
    assert _state_zero(work, m, n, k, 64, 32, 16)
