"""GPU tests of the reference C ABI (include/rocknpu.h) through host buffers,
mirroring how the ggml adapter calls it: every matmul entry point against
the oracle, grouping == separate calls, cache release/prewarm/stats, the
overlap callback, and the reference's error codes."""
import numpy as np
import pytest

from oracle import oracle as orc
from rocknpu_amd import hip, synth
from rocknpu_amd.capi import STATUS_INVALID_ARGUMENT, STATUS_OK, Context

pytestmark = pytest.mark.gpu


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ctx():
    c = Context()
    yield c
    c.close()


def _w8a8_ref(kind, blocks, a, n):
    return orc.matmul_q_w8a8(kind, blocks, a, n, threads=8)


@pytest.mark.parametrize("kind,m,k,n", [(4, 128, 2048, 5632), (4, 1, 2048, 256), (4, 7, 512, 96), (6, 16, 5632, 2048),
                                        (6, 1, 2048, 128), (5, 12, 1024, 64), (4, 300, 768, 200), (6, 4, 256, 33)])
def test_matmul_q_matches_oracle(ctx, kind, m, k, n):
    blocks = synth.kquant(kind, n, k, index=800 + kind + m + n)
    a = synth.activations(m, k, index=900 + m)
    out = np.empty((m, n), np.float32)
    assert ctx.matmul_q(kind, blocks, a, out, k, n) == STATUS_OK
    assert np.array_equal(_bits(out), _bits(_w8a8_ref(kind, blocks, a, n)))
    # second call hits the resident cache and gives the same bits
    out2 = np.empty_like(out)
    assert ctx.matmul_q(kind, blocks, a, out2, k, n) == STATUS_OK
    assert np.array_equal(_bits(out2), _bits(out))


def test_matmul_q_error_codes(ctx):
    k, n = 512, 32
    blocks = synth.q4_k(n, k, index=1)
    a = synth.activations(4, k, index=2)
    out = np.empty((4, n), np.float32)
    assert ctx.matmul_q(4, blocks[:-1], a, out, k, n) == STATUS_INVALID_ARGUMENT      # byte count
    assert ctx.matmul_q(4, blocks, a[:, :300].copy(), out, 300, n) == STATUS_INVALID_ARGUMENT  # k % 256
    bad = a.copy()
    bad[2, 17] = np.nan
    sentinel = np.full((4, n), 7.0, np.float32)
    assert ctx.matmul_q(4, blocks, bad, sentinel, k, n) == STATUS_INVALID_ARGUMENT   # non-finite row
    assert np.all(sentinel == 7.0)                                                     # output untouched
    bad[2, 17] = np.inf
    assert ctx.matmul_q(4, blocks, bad, out, k, n) == STATUS_INVALID_ARGUMENT
    assert ctx.matmul_q(5, synth.q5_k(n, k, index=3), a[:1].copy(), out[:1], k, n) == STATUS_INVALID_ARGUMENT  # Q5_K M=1
    # a weight whose dequantised row is non-finite is rejected, not cached
    wb = synth.q4_k(n, k, index=4).reshape(n, -1, 144).copy()
    wb[5, 0, 0:2] = [0x00, 0x7C]
    assert ctx.matmul_q(4, wb.reshape(-1), a, out, k, n) == STATUS_INVALID_ARGUMENT


def test_zero_activation_row_gives_zero_output(ctx):
    k, n = 512, 64
    blocks = synth.q6_k(n, k, index=5)
    a = synth.activations(3, k, index=6)
    a[1] = 0.0
    out = np.empty((3, n), np.float32)
    assert ctx.matmul_q(6, blocks, a, out, k, n) == STATUS_OK
    assert not out[1].any()
    assert np.array_equal(_bits(out), _bits(_w8a8_ref(6, blocks, a, n)))


def test_concat_pair_equal_separate_calls(ctx):
    m, k = 128, 2048
    ns = (2048, 256, 256)
    ws = [synth.q4_k(n, k, index=1000 + i) for i, n in enumerate(ns)]
    a = synth.activations(m, k, index=1100)
    outs = [np.empty((m, n), np.float32) for n in ns]
    assert ctx.matmul_q_concat(ws, [4, 4, 4], ns, a, outs, k) == STATUS_OK
    for w, n, o in zip(ws, ns, outs):
        assert np.array_equal(_bits(o), _bits(_w8a8_ref(4, w, a, n)))
    o1, o2 = np.empty((m, ns[1]), np.float32), np.empty((m, ns[2]), np.float32)
    assert ctx.matmul_q_pair_mtile(ws[1], 4, ns[1], ws[2], 4, ns[2], a, o1, o2, k) == STATUS_OK
    assert np.array_equal(_bits(o1), _bits(outs[1])) and np.array_equal(_bits(o2), _bits(outs[2]))
    # mixed kinds in a group
    w6 = synth.q6_k(96, k, index=1200)
    oa, ob = np.empty((m, 256), np.float32), np.empty((m, 96), np.float32)
    assert ctx.matmul_q_concat([ws[1], w6], [4, 6], [256, 96], a, [oa, ob], k) == STATUS_OK
    assert np.array_equal(_bits(ob), _bits(_w8a8_ref(6, w6, a, 96)))
    assert ctx.matmul_q_concat([ws[1]] * 5, [4] * 5, [256] * 5, a, [oa] * 5, k) == STATUS_INVALID_ARGUMENT


def test_m1_groups_and_w8a8_entries(ctx):
    k = 2048
    ns = (512, 128, 64)
    ws = [synth.q4_k(n, k, index=1300 + i) for i, n in enumerate(ns)]
    x = synth.activations(1, k, index=1400)
    refs = [_w8a8_ref(4, w, x, n)[0] for w, n in zip(ws, ns)]
    outs = [np.empty(n, np.float32) for n in ns]
    assert ctx.matmul_q_triple_m1(ws[0], 4, ns[0], ws[1], 4, ns[1], ws[2], 4, ns[2], x[0], *outs, k) == STATUS_OK
    for o, r in zip(outs, refs):
        assert np.array_equal(_bits(o), _bits(r))
    o1, o2 = np.empty(ns[0], np.float32), np.empty(ns[1], np.float32)
    assert ctx.matmul_q_pair_m1(ws[0], 4, ns[0], ws[1], 4, ns[1], x[0], o1, o2, k) == STATUS_OK
    assert np.array_equal(_bits(o1), _bits(refs[0])) and np.array_equal(_bits(o2), _bits(refs[1]))
    # caller-quantised W8 entries
    w8s = [orc.repack_w8(4, w, k, n) for w, n in zip(ws, ns)]
    o = np.empty(ns[0], np.float32)
    assert ctx.matmul_w8a8_m1(w8s[0][0], w8s[0][1], x[0], o, k, ns[0]) == STATUS_OK
    assert np.array_equal(_bits(o), _bits(refs[0]))
    o = np.empty(ns[0], np.float32)
    assert ctx.matmul_w8a8_m1_nsplit(w8s[0][0], w8s[0][1], x[0], o, k, ns[0], 96) == STATUS_OK
    assert np.array_equal(_bits(o), _bits(refs[0]))
    p1, p2 = np.empty(ns[0], np.float32), np.empty(ns[1], np.float32)
    assert ctx.matmul_w8a8_pair_m1(w8s[0][0], w8s[0][1], ns[0], w8s[1][0], w8s[1][1], ns[1], x[0], p1, p2,
                                   k) == STATUS_OK
    assert np.array_equal(_bits(p1), _bits(refs[0])) and np.array_equal(_bits(p2), _bits(refs[1]))
    t = [np.empty(n, np.float32) for n in ns]
    assert ctx.matmul_w8a8_triple_m1(w8s[0][0], w8s[0][1], ns[0], w8s[1][0], w8s[1][1], ns[1], w8s[2][0],
                                     w8s[2][1], ns[2], x[0], *t, k) == STATUS_OK
    for o, r in zip(t, refs):
        assert np.array_equal(_bits(o), _bits(r))
    a16 = synth.activations(16, k, index=1500)
    o16 = np.empty((16, ns[1]), np.float32)
    assert ctx.matmul_w8a8_m16(w8s[1][0], w8s[1][1], a16, o16, k, ns[1]) == STATUS_OK
    assert np.array_equal(_bits(o16), _bits(_w8a8_ref(4, ws[1], a16, ns[1])))
    bad_scales = w8s[1][1].copy()
    bad_scales[3] = 0.0
    assert ctx.matmul_w8a8_m1(w8s[1][0], bad_scales, x[0], np.empty(ns[1], np.float32), k,
                              ns[1]) == STATUS_INVALID_ARGUMENT


def test_swiglu_down(ctx):
    k, ffn, out_n = 512, 256, 128
    gw, uw = synth.q4_k(ffn, k, index=1600), synth.q4_k(ffn, k, index=1601)
    dw = synth.q4_k(out_n, ffn, index=1602)
    (g8, gs), (u8, us), (d8, ds) = (orc.repack_w8(4, gw, k, ffn), orc.repack_w8(4, uw, k, ffn),
                                    orc.repack_w8(4, dw, ffn, out_n))
    x = synth.activations(1, k, index=1603)
    out = np.empty(out_n, np.float32)
    assert ctx.matmul_w8a8_swiglu_down(g8, gs, u8, us, d8, ds, x[0], out, k, ffn, out_n) == STATUS_OK
    gate = _w8a8_ref(4, gw, x, ffn)[0]
    up = _w8a8_ref(4, uw, x, ffn)[0]
    # exp(-gate) overflows to inf for gate below about -88.7: 1 / (1 + inf) = 0
    # is then the sigmoid's correctly rounded f32 value, so the overflow is benign
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate))).astype(np.float32)
    h = (gate * sig * up).astype(np.float32)
    ref = _w8a8_ref(4, dw, h[None, :], out_n)[0]
    # SwiGLU's exp is the platform libm on both sides; allow its last-ulp freedom
    np.testing.assert_allclose(out, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())


def test_cache_stats_release_prewarm_overlap(ctx):
    k, n = 1024, 128
    w = synth.q4_k(n, k, index=1700)
    x = synth.activations(1, k, index=1701)
    before = ctx.decode_cache_stats()
    out = np.empty(n, np.float32)
    ran = []
    assert ctx.set_overlap(lambda: ran.append(1)) == STATUS_OK
    assert ctx.matmul_q(4, w, x, out, k, n) == STATUS_OK
    assert ran == [1]                                  # one-shot, run during the M=1 call
    assert ctx.matmul_q(4, w, x, out, k, n) == STATUS_OK
    assert ran == [1]
    after = ctx.decode_cache_stats()
    assert after.misses == before.misses + 1 and after.hits == before.hits + 1
    assert after.entries >= before.entries + 1 and after.resident_bytes > before.resident_bytes
    # prewarm fills the prompt cache; release drops it without touching decode caches
    assert ctx.prewarm_quantized_m16(w, 4, k, n) == STATUS_OK
    assert ctx.mtile_release([w]) == STATUS_OK
    assert ctx.decode_cache_stats().entries == after.entries
    a = synth.activations(4, k, index=1702)
    o4 = np.empty((4, n), np.float32)
    assert ctx.matmul_q(4, w, a, o4, k, n) == STATUS_OK
    assert np.array_equal(_bits(o4), _bits(_w8a8_ref(4, w, a, n)))
    assert ctx.mtile_release([]) == STATUS_INVALID_ARGUMENT


def test_decode_q8k_entry(ctx):
    for kind, k, n, m in ((4, 2048, 256, 1), (6, 5632, 128, 4), (4, 2048, 5632, 2)):
        w = synth.kquant(kind, n, k, index=1800 + kind + m)
        x = synth.activations(m, k, index=1900 + m)
        out = np.empty((m, n), np.float32)
        assert ctx.matmul_q_q8k(kind, w, x, out, k, n) == STATUS_OK
        q8 = orc.quantize_q8_k(x)
        ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=8)
        for mi in range(m):
            _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[mi])
            assert np.all(np.abs(out[mi].astype(np.float64) - ref[mi]) <= 1e-5 * mag)
    bad = synth.activations(1, 256, index=1)
    bad[0, 3] = np.inf
    assert ctx.matmul_q_q8k(4, synth.q4_k(8, 256, index=2), bad, np.empty((1, 8), np.float32), 256,
                            8) == STATUS_INVALID_ARGUMENT


def test_f16_bridge(ctx):
    m, k, n = 5, 96, 40
    g = np.random.default_rng(3)
    w = (g.standard_normal((n, k)) * 0.1).astype(np.float16)
    a = g.standard_normal((m, k)).astype(np.float32)
    out = np.empty((m, n), np.float32)
    assert ctx.matmul_f16(w.view(np.uint16), a, out, k, n) == STATUS_OK
    ref = a.astype(np.float16).astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("mode,k", [("1", 2048), ("all", 512), ("down", 5632), ("down", 2048)])
def test_prefill_hilo_matches_oracle(monkeypatch, mode, k):
    """ROCKNPU_PREFILL_HILO (lib.rs:2005-2083): the prompt-path W8A8 with the two-part
    activation encoding, bit for bit against the oracle's stack / W8A8 / sum. "down"
    applies only where K > 4096 or K is not a multiple of 512; elsewhere the plain route
    runs. M=1 never uses it."""
    monkeypatch.setenv("ROCKNPU_PREFILL_HILO", mode)
    c = Context()
    keep = []  # weights stay alive (and at their addresses) for the context's lifetime, as the ABI requires
    try:
        m, n = 12, 96
        for kind in (4, 6):
            blocks = synth.kquant(kind, n, k, index=1300 + kind + k)
            keep.append(blocks)
            a = synth.activations(m, k, index=1310 + k)
            out = np.empty((m, n), np.float32)
            assert c.matmul_q(kind, blocks, a, out, k, n) == STATUS_OK
            applies = mode != "down" or k > 4096 or k % 512 != 0
            ref = orc.matmul_q_hilo(kind, blocks, a, n, threads=8) if applies else _w8a8_ref(kind, blocks, a, n)
            assert np.array_equal(_bits(out), _bits(ref)), (kind, mode, k)
        # concat-N entry uses it too
        ws = [synth.q4_k(nn, k, index=1320 + nn) for nn in (64, 32)]
        keep.extend(ws)
        outs = [np.empty((m, nn), np.float32) for nn in (64, 32)]
        assert c.matmul_q_concat(ws, [4, 4], [64, 32], a, outs, k) == STATUS_OK
        for w, nn, o in zip(ws, (64, 32), outs):
            ref = orc.matmul_q_hilo(4, w, a, nn, threads=8) if applies else _w8a8_ref(4, w, a, nn)
            assert np.array_equal(_bits(o), _bits(ref))
        # one row: the decode route, no two-part encoding
        out1 = np.empty((1, n), np.float32)
        blocks = synth.q4_k(n, k, index=1330)
        keep.append(blocks)
        assert c.matmul_q(4, blocks, a[:1].copy(), out1, k, n) == STATUS_OK
        assert np.array_equal(_bits(out1), _bits(_w8a8_ref(4, blocks, a[:1], n)))
    finally:
        c.close()


def test_w8_sidecar_get_converts_writes_and_reloads(tmp_path):
    """rocknpu_w8_sidecar_get: a miss converts on the GPU (the oracle's repack, bit for
    bit) and writes the sidecar; the next call is served from the files; a changed
    source is converted again, not served stale; manifest of a directory of tensors."""
    from rocknpu_amd import sidecar

    c = Context()
    try:
        for kind, n, k in ((4, 40, 1024), (6, 33, 512), (5, 16, 256)):
            blocks = synth.kquant(kind, n, k, index=1400 + kind)
            w_ref, s_ref = orc.repack_w8(kind, blocks, k, n)
            name = f"blk.0.q{kind}.weight"
            st, w8, sc, hit = sidecar.get(c, tmp_path, name, kind, blocks, k, n, write_back=True)
            assert st == STATUS_OK and not hit
            assert np.array_equal(w8, w_ref) and np.array_equal(_bits(sc), _bits(s_ref))
            st, w8b, scb, hit = sidecar.get(c, tmp_path, name, kind, blocks, k, n)
            assert st == STATUS_OK and hit
            assert np.array_equal(w8b, w_ref) and np.array_equal(_bits(scb), _bits(s_ref))
            changed = blocks.copy()
            changed.reshape(n, -1)[0, -1] ^= 0x11
            st, w8c, _, hit = sidecar.get(c, tmp_path, name, kind, changed, k, n)
            assert st == STATUS_OK and not hit
            assert np.array_equal(w8c, orc.repack_w8(kind, changed, k, n)[0])
        # no directory: conversion only
        blocks = synth.q4_k(8, 256, index=1410)
        st, w8, _, hit = sidecar.get(c, None, "x", 4, blocks, 256, 8)
        assert st == STATUS_OK and not hit and np.array_equal(w8, orc.repack_w8(4, blocks, 256, 8)[0])
        tensors = {f"blk.{i}.ffn_gate.weight": (4, synth.q4_k(16, 512, index=1420 + i), 512, 16) for i in range(3)}
        man = sidecar.make_directory(c, tmp_path / "dir", tensors, "synthetic")
        assert man["format"] == "rocknpu-w8-sidecar-v2" and len(man["tensors"]) == 3
        for name, (kind, blocks, k, n) in tensors.items():
            assert man["tensors"][name]["source_sample_fnv1a64"] == f"{orc.source_fingerprint(blocks):016x}"
            assert sidecar.read(tmp_path / "dir", name, blocks, k, n) is not None
    finally:
        c.close()


@pytest.mark.parametrize("k", [1024, 2048])
def test_decode_cache_stats_count_the_q8k_route(k):
    """The Q8_K decode route's resident raw blocks are decode-cache entries:
    entries, resident bytes, hits and misses move with its calls. A weight the
    one-row rule reads tiled (8-block rows here; 4-block rows stay raw) also
    holds its tiled copy."""
    n = 96
    tiled = k == 2048
    assert all(hip.gemv_tiled_preferred(kind, 1, k) == tiled for kind in (4, 6))
    t4 = hip.gemv_tiled_bytes(4, k, n) if tiled else 0
    t6 = hip.gemv_tiled_bytes(6, k, n) if tiled else 0
    w4 = synth.q4_k(n, k, index=1720)
    w6 = synth.q6_k(n, k, index=1721)
    x = synth.activations(1, k, index=1722)
    out = np.empty((1, n), np.float32)
    with Context() as c:
        s0 = c.decode_cache_stats()
        assert (s0.entries, s0.resident_bytes, s0.hits, s0.misses) == (0, 0, 0, 0)
        assert c.matmul_q_q8k(4, w4, x, out, k, n) == STATUS_OK
        s1 = c.decode_cache_stats()
        assert (s1.entries, s1.resident_bytes, s1.misses, s1.hits) == (1, w4.nbytes + t4, 1, 0)
        assert c.matmul_q_q8k(4, w4, x, out, k, n) == STATUS_OK
        s2 = c.decode_cache_stats()
        assert (s2.entries, s2.resident_bytes, s2.misses, s2.hits) == (1, w4.nbytes + t4, 1, 1)
        outs = [np.empty((1, n), np.float32) for _ in range(2)]
        assert c.matmul_q_q8k_group([w4, w6], [4, 6], [n, n], x, outs, k) == STATUS_OK
        s3 = c.decode_cache_stats()
        assert (s3.entries, s3.resident_bytes, s3.misses, s3.hits) == (2, w4.nbytes + t4 + w6.nbytes + t6, 2, 1)
        assert s3.miss_ns > 0 and s3.hit_ns > 0 and s3.worker1_calls == 3


def test_w8a8_rejects_k_beyond_exact_int32():
    """127 * 127 * K must stay below 2^31 for exact int32 sums: K = 133376 is refused
    before any weight is uploaded, on every W8A8 entry."""
    k, n = 133376, 2
    w = synth.q4_k(n, k, index=1730)
    a = synth.activations(2, k, index=1731)
    out = np.zeros((2, n), np.float32)
    with Context() as c:
        assert c.matmul_q(4, w, a, out, k, n) == STATUS_INVALID_ARGUMENT
        assert c.matmul_q(4, w, a[:1].copy(), out[:1], k, n) == STATUS_INVALID_ARGUMENT
        s = c.decode_cache_stats()
        assert s.entries == 0 and s.misses == 0
    assert not out.any()


def test_gemv_stall_gives_nan_and_execution_error():
    """The fused lane-per-block decode GEMV waits for its workgroup's quantising
    waves with a bounded poll. Forced from the host to give up (test hook: one
    arrival more than the workgroup has, 8 polls; every wave still exits), each
    output is NaN, the stall flag is set once, and the C ABI's fused decode entry
    returns ROCKNPU_STATUS_EXECUTION_ERROR. With the hook off the same calls
    match the oracle and leave the flag clear. A context of its own: the weight
    caches are keyed by host address, which freed arrays of other tests reuse."""
    import ctypes

    import torch

    from rocknpu_amd import _lib, hip
    from rocknpu_amd.capi import STATUS_EXECUTION_ERROR

    kind, ns, k, m = 4, (256, 512), 1024, 1
    assert not hip.gemv_tiled_preferred(kind, m, k)  # the C ABI reads the raw rows
    mf, lanes, waves = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    arr = (ctypes.c_size_t * 2)(*ns)
    assert _lib.load().rocknpu_hip_gemv_shape(kind, m, k, arr, 2, 1, 0, ctypes.byref(mf), ctypes.byref(lanes),
                                              ctypes.byref(waves)) == 0
    assert mf.value == 0  # the lane-per-block kernel, the one with the wait
    ws = [synth.kquant(kind, n, k, index=2300 + i) for i, n in enumerate(ns)]
    x = synth.activations(m, k, index=2310)
    dws = [torch.from_numpy(w).to("cuda") for w in ws]
    dx = torch.from_numpy(x).to("cuda")
    torch.cuda.synchronize()
    assert not hip.gemv_take_stall()
    ctx = Context()
    print("stall hook on: launch layer", flush=True)
    hip.gemv_test_stall(8)
    try:
        outs = hip.gemv_q_f32(kind, dws, k, ns, dx)
        torch.cuda.synchronize()
        assert all(np.isnan(o.cpu().numpy()).all() for o in outs)
        assert hip.gemv_take_stall()
        assert not hip.gemv_take_stall()  # taking clears it
        print("stall hook on: C ABI", flush=True)
        houts = [np.zeros((m, n), np.float32) for n in ns]
        assert ctx.matmul_q_q8k_group(ws, [kind, kind], ns, x, houts, k) == STATUS_EXECUTION_ERROR
        assert not hip.gemv_take_stall()
    finally:
        hip.gemv_test_stall(0)
    print("stall hook off", flush=True)
    houts = [np.zeros((m, n), np.float32) for n in ns]
    assert ctx.matmul_q_q8k_group(ws, [kind, kind], ns, x, houts, k) == STATUS_OK
    ctx.close()
    outs = hip.gemv_q_f32(kind, dws, k, ns, dx)
    torch.cuda.synchronize()
    assert not hip.gemv_take_stall()
    q8 = orc.quantize_q8_k(x)
    for w, n, o, h in zip(ws, ns, outs, houts):
        assert np.array_equal(_bits(o.cpu().numpy()), _bits(h))
        ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=8)
        _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[0])
        assert np.all(np.abs(h[0].astype(np.float64) - ref[0]) <= 1e-5 * mag)


def test_swiglu_down_caches_counts_and_rejects_nonfinite():
    """The device-side SwiGLU path keeps the reference's bookkeeping: two decode
    calls per invocation (the pair and the down projection), misses then hits
    on the decode caches, the same output on a repeat, and a non-finite
    activation rejected with the output buffer left as it was."""
    k, ffn, out_n = 1024, 512, 256
    ws = [synth.q4_k(n, kk, index=2400 + i) for i, (n, kk) in enumerate(((ffn, k), (ffn, k), (out_n, ffn)))]
    (g8, gs), (u8, us), (d8, ds) = (orc.repack_w8(4, ws[0], k, ffn), orc.repack_w8(4, ws[1], k, ffn),
                                    orc.repack_w8(4, ws[2], ffn, out_n))
    x = synth.activations(1, k, index=2410)[0]
    with Context() as c:
        out1 = np.zeros(out_n, np.float32)
        assert c.matmul_w8a8_swiglu_down(g8, gs, u8, us, d8, ds, x, out1, k, ffn, out_n) == STATUS_OK
        st1 = c.decode_cache_stats()
        assert (st1.hits, st1.misses) == (0, 2)
        out2 = np.zeros(out_n, np.float32)
        assert c.matmul_w8a8_swiglu_down(g8, gs, u8, us, d8, ds, x, out2, k, ffn, out_n) == STATUS_OK
        st2 = c.decode_cache_stats()
        assert (st2.hits, st2.misses) == (2, 2)
        assert np.array_equal(_bits(out1), _bits(out2))
        bad = x.copy()
        bad[7] = np.nan
        out3 = np.full(out_n, 3.0, np.float32)
        assert c.matmul_w8a8_swiglu_down(g8, gs, u8, us, d8, ds, bad, out3, k, ffn, out_n) == STATUS_INVALID_ARGUMENT
        assert np.all(out3 == 3.0)
