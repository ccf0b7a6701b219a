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
