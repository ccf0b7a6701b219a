"""MUL_MAT routing (include/rocknpu_route.h) on the CPU: which nodes the
backend takes (supports_op, adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:614-715)
and the same-input groups (rocknpu_mtile_group, :856-976). Host logic only: no
node here is run."""
import numpy as np
import pytest

from rocknpu_amd import route as R
from rocknpu_amd import synth


def _blocks(wt, n, k):
    if wt == R.F16:
        return np.zeros((n, k), np.uint16)
    return np.zeros(n * (k // 256) * R.BLOCK_BYTES[wt], np.uint8)


def _node(wt=R.Q4_K, n=64, k=512, m=8, x=None, **kw):
    x = np.zeros((m, k), np.float32) if x is None else x
    out = np.zeros((x.shape[0], n), np.float32)
    w = _blocks(wt, n, k)
    nd = R.node(wt, w, k, n, x, out, **kw)
    nd._keep = (w, x, out)  # the arrays outlive the node
    return nd


@pytest.mark.parametrize("wt", [R.Q4_K, R.Q5_K, R.Q6_K, R.F16])
def test_prompt_nodes_supported(wt):
    assert R.supported(_node(wt, m=8))
    assert R.supported(_node(wt, m=513, n=40, k=768))   # no NPU tile limits on the GPU


def test_decode_routes():
    # M = 1 stays on the CPU by default (ggml-rocknpu.cpp:674-679); the GPU
    # routes take Q4_K and Q6_K, never Q5_K (lib.rs:5300) or F16 (:696-698)
    for wt in (R.Q4_K, R.Q6_K):
        assert not R.supported(_node(wt, m=1), R.DECODE_CPU)
        assert R.supported(_node(wt, m=1), R.DECODE_GGML)
        assert R.supported(_node(wt, m=1), R.DECODE_W8A8)
    for wt in (R.Q5_K, R.F16):
        for d in (R.DECODE_CPU, R.DECODE_GGML, R.DECODE_W8A8):
            assert not R.supported(_node(wt, m=1), d)


def test_rejections_follow_supports_op():
    # ggml-rocknpu.cpp:620-637: types, contiguity, 2-D, matching K
    assert not R.supported(_node(R.Q4_K, activation_type=R.F16))
    assert not R.supported(_node(R.Q4_K, output_type=R.F16))
    assert not R.supported(_node(R.Q4_K, contiguous=False))
    nd = _node(R.Q4_K)
    nd.weight_ne[2] = 2
    assert not R.supported(nd)
    nd = _node(R.Q4_K)
    nd.activation_ne[3] = 2
    assert not R.supported(nd)
    nd = _node(R.Q4_K)
    nd.activation_ne[0] = 256
    assert not R.supported(nd)
    # K-quant K must be whole super-blocks, and the weight bytes must match the shape
    x = np.zeros((4, 320), np.float32)
    nd = R.node(R.Q4_K, np.zeros(64 * 144, np.uint8), 320, 64, x, np.zeros((4, 64), np.float32))
    assert not R.supported(nd)
    nd = _node(R.Q6_K)
    nd.weight_bytes -= 210
    assert not R.supported(nd)
    nd = _node(R.F16)
    nd.weight_bytes += 2
    assert not R.supported(nd)
    nd = _node(R.Q4_K)
    nd.output = None
    assert not R.supported(nd)
    # an unknown weight type (ggml Q4_0 = 2)
    nd = _node(R.Q4_K)
    nd.weight_type = 2
    assert not R.supported(nd)


def _layer(m, k=512, ffn=1024):
    """A transformer layer's projections, in graph order, with their shared inputs."""
    xa, xo, xf = (np.zeros((m, k), np.float32) for _ in range(3))
    xd = np.zeros((m, ffn), np.float32)
    return [
        _node(R.Q4_K, 64, k, x=xa), _node(R.Q4_K, 32, k, x=xa), _node(R.Q6_K, 32, k, x=xa),  # q, k, v
        _node(R.Q4_K, 64, k, x=xo),                                                         # o
        _node(R.Q4_K, ffn, k, x=xf), _node(R.Q4_K, ffn, k, x=xf),                           # gate, up
        _node(R.Q6_K, k, ffn, x=xd),                                                        # down
    ]


@pytest.mark.parametrize("m,decode", [(8, R.DECODE_CPU), (1, R.DECODE_GGML), (1, R.DECODE_W8A8)])
def test_plan_groups_a_layer(m, decode):
    groups, lead = R.plan(_layer(m), decode)
    assert groups == 4
    assert lead == [0, 0, 0, 3, 4, 4, 6]


def test_plan_decode_on_cpu_takes_nothing():
    groups, lead = R.plan(_layer(1), R.DECODE_CPU)
    assert groups == 0 and lead == [-1] * 7


def test_plan_interleaved_inputs_and_group_limit():
    xa, xf = np.zeros((4, 512), np.float32), np.zeros((4, 512), np.float32)
    nodes = [_node(x=xa), _node(x=xf), _node(x=xa), _node(x=xf), _node(x=xa)]
    assert R.plan(nodes) == (2, [0, 1, 0, 1, 0])
    # at most 4 per group; the rest lead a group of their own
    same = [_node(x=xa) for _ in range(6)]
    assert R.plan(same) == (2, [0, 0, 0, 0, 4, 4])


def test_plan_keeps_mismatches_apart():
    x = np.zeros((4, 1024), np.float32)
    # another K on the same input, another M seen through the same pointer,
    # Q5_K and F16 (the concat entry takes Q4_K/Q6_K only), an unsupported node
    a = _node(R.Q4_K, 64, 1024, x=x)
    b = _node(R.Q4_K, 64, 512, x=x[:, :512].copy())
    b.activations = a.activations
    c = _node(R.Q4_K, 64, 1024, x=x[:2])
    c.activations = a.activations
    d = _node(R.Q5_K, 64, 1024, x=x)
    e = _node(R.F16, 64, 1024, x=x)
    f = _node(R.Q4_K, 64, 1024, x=x, contiguous=False)
    g = _node(R.Q6_K, 64, 1024, x=x)
    groups, lead = R.plan([a, b, c, d, e, f, g])
    assert lead == [0, 1, 2, 3, 4, -1, 0]
    assert groups == 5


def test_plan_of_synthetic_weights_matches_shapes():
    # real block data does not change the plan
    k, n = 512, 48
    x = synth.activations(3, k, index=5)
    nodes = []
    for i, wt in enumerate((R.Q4_K, R.Q6_K)):
        w = synth.kquant(4 if wt == R.Q4_K else 6, n, k, index=i)
        out = np.zeros((3, n), np.float32)
        nd = R.node(wt, w, k, n, x, out)
        nd._keep = (w, out)
        nodes.append(nd)
    assert R.plan(nodes) == (1, [0, 0])


def _out_node(wt, n, k, x, out, name=None):
    """A node whose output array is given (so tests can make outputs alias inputs)."""
    w = _blocks(wt, n, k)
    nd = R.node(wt, w, k, n, x, out, name=name)
    nd._keep = (w, x, out)
    return nd


def test_plan_does_not_move_a_member_past_a_writer_of_its_input():
    # [A: reads X; C: writes X (a buffer ggml-alloc reused); B: reads X]: B reads
    # C's output, so it must run after C and cannot join A's group
    m, k = 4, 512
    x, y = np.zeros((m, k), np.float32), np.zeros((m, k), np.float32)
    a = _out_node(R.Q4_K, 64, k, x, np.zeros((m, 64), np.float32))
    c = _out_node(R.Q4_K, k, k, y, x)          # N = K: its output is exactly X
    b = _out_node(R.Q4_K, 64, k, x, np.zeros((m, 64), np.float32))
    assert R.plan([a, c, b]) == (3, [0, 1, 2])
    # a writer of only part of X is a conflict too
    part = x.reshape(-1)[k:k + 32 * 2].reshape(2, 32)
    c2 = _out_node(R.Q4_K, 32, k, np.zeros((2, k), np.float32), part)
    assert R.plan([a, c2, b]) == (3, [0, 1, 2])


def test_plan_does_not_move_a_member_past_a_reader_or_writer_of_its_output():
    m, k = 4, 512
    x, z = np.zeros((m, k), np.float32), np.zeros((m, k), np.float32)
    a = _out_node(R.Q4_K, 64, k, x, np.zeros((m, 64), np.float32))
    t_reads_z = _out_node(R.Q4_K, 64, k, z, np.zeros((m, 64), np.float32))
    b_writes_z = _out_node(R.Q4_K, k, k, x, z)   # B's output is T's input
    assert R.plan([a, t_reads_z, b_writes_z]) == (3, [0, 1, 2])
    w = np.zeros((m, 64), np.float32)
    t_writes_w = _out_node(R.Q4_K, 64, k, z, w)
    b_writes_w = _out_node(R.Q4_K, 64, k, x, w)  # both write W: the later write must stay last
    assert R.plan([a, t_writes_w, b_writes_w]) == (3, [0, 1, 2])


def test_plan_groups_across_unrelated_nodes_and_rejects_self_aliasing_members():
    m, k = 4, 512
    x = np.zeros((m, k), np.float32)
    a = _out_node(R.Q4_K, 64, k, x, np.zeros((m, 64), np.float32))
    t = _out_node(R.Q4_K, 64, k, np.zeros((m, k), np.float32), np.zeros((m, 64), np.float32))
    b = _out_node(R.Q4_K, 64, k, x, np.zeros((m, 64), np.float32))
    assert R.plan([a, t, b]) == (2, [0, 1, 0])
    # a member writing the shared input, or the output of an earlier member
    b_in_place = _out_node(R.Q4_K, k, k, x, x)
    assert R.plan([a, b_in_place]) == (2, [0, 1])
    shared = np.zeros((m, 64), np.float32)
    a2 = _out_node(R.Q4_K, 64, k, x, shared)
    b2 = _out_node(R.Q4_K, 64, k, x, shared)
    assert R.plan([a2, b2]) == (2, [0, 1])


def test_plan_grouping_switch(monkeypatch):
    monkeypatch.setenv("ROCKNPU_MTILE_GROUP", "0")
    groups, lead = R.plan(_layer(8))
    assert groups == 7 and lead == list(range(7))
    monkeypatch.setenv("ROCKNPU_MTILE_GROUP", "1")
    assert R.plan(_layer(8))[1] == [0, 0, 0, 3, 4, 4, 6]


def test_route_stats_need_a_context():
    import ctypes
    from rocknpu_amd import _lib
    st = R.RouteStats()
    assert _lib.load().rocknpu_route_stats_get(None, ctypes.byref(st)) == -1
