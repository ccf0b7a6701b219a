"""GPU tests of the MUL_MAT routing (include/rocknpu_route.h): a layer's
projections run through rocknpu_route_run, grouped by shared input, give
bit-for-bit the outputs of one direct entry-point call per projection; and the
grouped decode entry equals the single decode entry."""
import numpy as np
import pytest

from rocknpu_amd import route as R
from rocknpu_amd import synth
from rocknpu_amd.capi import Context

pytestmark = pytest.mark.gpu

TYPE = {4: R.Q4_K, 6: R.Q6_K}


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _layer(m, k=512, ffn=768, seed=0):
    """(kind, n, k, input tag) per projection, graph order: q, k, v, o, gate, up, down."""
    spec = [(4, 64, k, "attn"), (4, 32, k, "attn"), (6, 32, k, "attn"), (4, 64, k, "o"),
            (4, ffn, k, "ffn"), (6, ffn, k, "ffn"), (6, k, ffn, "down")]
    inputs = {tag: synth.activations(m, kk, index=seed * 10 + i)
              for i, (tag, kk) in enumerate((("attn", k), ("o", k), ("ffn", k), ("down", ffn)))}
    weights = [synth.kquant(kind, n, kk, index=seed * 100 + i) for i, (kind, n, kk, _) in enumerate(spec)]
    return spec, inputs, weights


@pytest.mark.parametrize("m,decode", [(1, R.DECODE_GGML), (1, R.DECODE_W8A8), (6, R.DECODE_CPU),
                                      (37, R.DECODE_GGML)])
def test_route_run_matches_direct_calls(m, decode):
    print(f"route m={m} decode={decode}", flush=True)
    spec, inputs, weights = _layer(m, seed=m)
    outs = [np.zeros((m, n), np.float32) for (_, n, _, _) in spec]
    nodes = [R.node(TYPE[kind], w, kk, n, inputs[tag], o)
             for (kind, n, kk, tag), w, o in zip(spec, weights, outs)]
    assert R.plan(nodes, decode)[1] == [0, 0, 0, 3, 4, 4, 6]
    with Context() as ctx:
        assert R.run(ctx, nodes, decode) == 0
        for (kind, n, kk, tag), w, got in zip(spec, weights, outs):
            ref = np.zeros((m, n), np.float32)
            if m == 1 and decode == R.DECODE_GGML:
                assert ctx.matmul_q_q8k(kind, w, inputs[tag], ref, kk, n) == 0
            else:
                assert ctx.matmul_q(kind, w, inputs[tag], ref, kk, n) == 0
            assert np.array_equal(_bits(got), _bits(ref)), (kind, n, tag)


def test_route_run_rejects_unsupported_and_decode_on_cpu():
    spec, inputs, weights = _layer(1)
    outs = [np.zeros((1, n), np.float32) for (_, n, _, _) in spec]
    nodes = [R.node(TYPE[kind], w, kk, n, inputs[tag], o)
             for (kind, n, kk, tag), w, o in zip(spec, weights, outs)]
    with Context() as ctx:
        # M = 1 nodes are not the backend's on the CPU decode route: the graph fails
        assert R.run(ctx, nodes, R.DECODE_CPU) == -1
        assert not any(o.any() for o in outs)
        assert R.run(ctx, [], R.DECODE_GGML) == 0


@pytest.mark.parametrize("m", [1, 3, 9])
def test_q8k_group_entry_equals_single_entry(m):
    k = 1024
    kinds, ns = [4, 6, 4, 6], [48, 40, 96, 16]
    x = synth.activations(m, k, index=70 + m)
    ws = [synth.kquant(kind, n, k, index=700 + i) for i, (kind, n) in enumerate(zip(kinds, ns))]
    outs = [np.zeros((m, n), np.float32) for n in ns]
    with Context() as ctx:
        assert ctx.matmul_q_q8k_group(ws, kinds, ns, x, outs, k) == 0
        for kind, n, w, got in zip(kinds, ns, ws, outs):
            ref = np.zeros((m, n), np.float32)
            assert ctx.matmul_q_q8k(kind, w, x, ref, k, n) == 0
            assert np.array_equal(_bits(got), _bits(ref))
        # argument guards: no members, five members, a mismatched byte count
        assert ctx.matmul_q_q8k_group([], [], [], x, [], k) == -1
        assert ctx.matmul_q_q8k_group(ws + ws[:1], kinds + [4], ns + [48], x, outs + outs[:1], k) == -1
        assert ctx.matmul_q_q8k_group([ws[0][:-1]], [4], [48], x, outs[:1], k) == -1


def test_route_run_keeps_order_when_a_buffer_is_reused():
    """[A reads X; C writes X; B reads X]: B must see C's output, as in graph
    order, so the result equals direct calls made in node order."""
    print("route alias", flush=True)
    m, k = 5, 512
    x = synth.activations(m, k, index=81)
    y = synth.activations(m, k, index=82)
    wa, wc, wb = (synth.kquant(4, n, k, index=810 + i) for i, n in enumerate((64, k, 48)))
    oa, ob = np.zeros((m, 64), np.float32), np.zeros((m, 48), np.float32)
    x_run = x.copy()
    nodes = [R.node(R.Q4_K, wa, k, 64, x_run, oa), R.node(R.Q4_K, wc, k, k, y, x_run),
             R.node(R.Q4_K, wb, k, 48, x_run, ob)]
    assert R.plan(nodes)[1] == [0, 1, 2]
    with Context() as ctx:
        assert R.run(ctx, nodes) == 0
        ra, rc, rb = np.zeros((m, 64), np.float32), np.zeros((m, k), np.float32), np.zeros((m, 48), np.float32)
        assert ctx.matmul_q(4, wa, x, ra, k, 64) == 0
        assert ctx.matmul_q(4, wc, y, rc, k, k) == 0
        assert ctx.matmul_q(4, wb, rc, rb, k, 48) == 0   # B reads what C wrote
    assert np.array_equal(_bits(oa), _bits(ra))
    assert np.array_equal(_bits(x_run), _bits(rc))
    assert np.array_equal(_bits(ob), _bits(rb))


def test_qkv_stash_across_separate_calls():
    """Layer 3's Q, then its K and V in a later call (another split): Q runs as
    one Q+K+V concat call with K/V kept in the context, K and V are served from
    that stash, and every output equals its direct call bit for bit
    (ggml-rocknpu.cpp:871-928)."""
    print("route qkv stash", flush=True)
    m, k = 40, 1024
    spec = (("q", 4, 128), ("k", 4, 32), ("v", 6, 32))
    ws = {name: synth.kquant(kind, n, k, index=830 + i) for i, (name, kind, n) in enumerate(spec)}
    x = synth.activations(m, k, index=84)

    def nodes_for(names, outs, act):
        return [R.node(TYPE[kind], ws[name], k, n, act, outs[name], name=f"blk.3.attn_{name}.weight")
                for name, kind, n in spec if name in names]

    with Context() as ctx:
        ref = {}
        for name, kind, n in spec:
            ref[name] = np.zeros((m, n), np.float32)
            assert ctx.matmul_q(kind, ws[name], x, ref[name], k, n) == 0
        # first pass: Q, K and V in one call (one same-input group); K/V weights become known
        outs = {name: np.zeros((m, n), np.float32) for name, _, n in spec}
        assert R.run(ctx, nodes_for("qkv", outs, x)) == 0
        st0 = R.stats(ctx)
        assert st0["mtile_group_calls"] == 1 and st0["qkv_triple_calls"] == 0
        # second pass: Q alone, then K and V in another call
        outs = {name: np.zeros((m, n), np.float32) for name, _, n in spec}
        assert R.run(ctx, nodes_for("q", outs, x)) == 0
        st1 = R.stats(ctx)
        assert st1["qkv_triple_calls"] == 1 and not outs["k"].any() and not outs["v"].any()
        assert R.run(ctx, nodes_for("kv", outs, x)) == 0
        st2 = R.stats(ctx)
        assert st2["qkv_stash_hits"] == 2 and st2["mtile_group_calls"] == st1["mtile_group_calls"]
        for name, _, _ in spec:
            assert np.array_equal(_bits(outs[name]), _bits(ref[name])), name
        # K/V of another input are computed, not served from the stash
        x2 = synth.activations(m, k, index=85)
        outs2 = {name: np.zeros((m, n), np.float32) for name, _, n in spec}
        assert R.run(ctx, nodes_for("q", outs2, x)) == 0
        assert R.run(ctx, nodes_for("kv", outs2, x2)) == 0
        assert R.stats(ctx)["qkv_stash_hits"] == 2
        for name, kind, n in spec[1:]:
            r2 = np.zeros((m, n), np.float32)
            assert ctx.matmul_q(kind, ws[name], x2, r2, k, n) == 0
            assert np.array_equal(_bits(outs2[name]), _bits(r2)), name


def test_split_profile(monkeypatch, capfd):
    """ROCKNPU_SPLIT_PROFILE (ggml-rocknpu.cpp:758-818, :1080-1092,
    :1623-1632): calls, nodes and the M buckets in the stats; at destroy one
    SHAPE PROFILE line per single projection shape timed after the 111
    warm-up calls, and the SPLIT PROFILE line whose first-111/rest and
    quarter times add up to the total."""
    import re
    monkeypatch.setenv("ROCKNPU_SPLIT_PROFILE", "1")
    k, calls = 256, 115
    xa, xg, xd = (synth.activations(m, k, index=7000 + m) for m in (4, 5, 8))
    wa, wb, wc, wd = (synth.kquant(kind, n, k, index=7010 + i) for i, (kind, n) in
                      enumerate(((4, 32), (4, 48), (6, 16), (6, 64))))
    outs = [np.zeros((m, n), np.float32) for m, n in ((4, 32), (5, 48), (5, 16), (8, 64))]
    nodes = [R.node(R.Q4_K, wa, k, 32, xa, outs[0]),          # alone, M = 4
             R.node(R.Q4_K, wb, k, 48, xg, outs[1]),          # a same-input pair, M = 5
             R.node(R.Q6_K, wc, k, 16, xg, outs[2]),
             R.node(R.Q6_K, wd, k, 64, xd, outs[3])]          # alone, M = 8
    with Context() as ctx:
        for i in range(calls):
            if i % 20 == 0:
                print(f"split profile call {i}", flush=True)
            assert R.run(ctx, nodes, R.DECODE_GGML) == 0
        s = R.stats(ctx)
        assert (s["graph_calls"], s["graph_nodes"]) == (calls, 4 * calls)
        assert (s["m4_mul_mat"], s["m8_mul_mat"], s["m12_mul_mat"], s["m16_mul_mat"], s["m_other_mul_mat"]) == \
            (calls, calls, 0, 0, 2 * calls)
        assert s["graph_ns"] > 0
        capfd.readouterr()
    err = capfd.readouterr().err
    shapes = re.findall(r"ROCKNPU SHAPE PROFILE M=(\d+) K=(\d+) N=(\d+) calls=(\d+)", err)
    assert sorted(shapes) == sorted([("4", "256", "32", str(calls - 111)), ("8", "256", "64", str(calls - 111))])
    line = re.search(r"ROCKNPU SPLIT PROFILE (.*)", err).group(1)
    f = dict(kv.split("=", 1) for kv in line.split())
    assert (f["graph_calls"], f["graph_nodes"], f["q4"], f["q6"]) == (str(calls), str(4 * calls), str(2 * calls),
                                                                      str(2 * calls))
    assert f["m"] == f"[4:{calls},8:{calls},12:0,16:0,other:{2 * calls}]"
    total = float(f["graph_ms"])
    assert abs(float(f["first111_ms"]) + float(f["rest_ms"]) - total) <= 0.01 + 1e-3 * total
    assert abs(sum(float(v) for v in f["q_ms"].strip("[]").split(",")) - total) <= 0.01 + 1e-3 * total
    assert 0 <= int(f["slow20"]) <= int(f["slow5"]) <= calls and float(f["max_ms"]) <= total


def test_no_split_profile_without_the_variable(monkeypatch, capfd):
    monkeypatch.delenv("ROCKNPU_SPLIT_PROFILE", raising=False)
    x = synth.activations(4, 256, index=7100)
    w = synth.kquant(4, 32, 256, index=7101)
    out = np.zeros((4, 32), np.float32)
    with Context() as ctx:
        assert R.run(ctx, [R.node(R.Q4_K, w, 256, 32, x, out)], R.DECODE_GGML) == 0
        assert R.stats(ctx)["m4_mul_mat"] == 1
    assert "SPLIT PROFILE" not in capfd.readouterr().err
