"""Seeded random shapes through the routed kernels, against the oracle: the
W8A8 GEMM (every route the shape takes, K splits included) bit-exact in int32
and f32, and the fused decode GEMV (1..16 activation rows, 1..3 projections
sharing them) within 1e-5 of the summed block-term magnitude. The shapes are
drawn once from a fixed seed, so a failure names a reproducible case."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rocknpu_amd import hip, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _gemm_shapes(count=48, seed=2024):
    """M across every route's range (the weight stream, 64-, 128- and 256-row
    tiles), N up to 12000, K a multiple of 64, at most 3e9 multiply-adds."""
    g = np.random.default_rng(seed)
    out = []
    bands = [(1, 17), (17, 65), (65, 129), (129, 257), (257, 1100)]
    while len(out) < count:
        lo, hi = bands[len(out) % len(bands)]
        m = int(g.integers(lo, hi))
        n = int(g.integers(1, 12000))
        k = 64 * int(g.integers(1, 97))
        while m * n * k > 3_000_000_000 and k > 64:
            k -= 64
        out.append((m, n, k))
    return out


@pytest.mark.parametrize("m,n,k", _gemm_shapes())
def test_gemm_random_shape_bit_exact(m, n, k):
    print(f"random gemm m={m} n={n} k={k} route={hip.gemm_workspace(m, n, k)}", flush=True)
    g = np.random.default_rng(m * 131 + n * 7 + k)
    a8 = g.integers(-127, 128, (m, k), dtype=np.int8)
    w8 = g.integers(-127, 128, (n, k), dtype=np.int8)
    as_ = (g.random(m, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    ws = (g.random(n, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    c = torch.empty((m, n), dtype=torch.int32, device=DEV)
    out = hip.gemm_w8a8(*(torch.from_numpy(x).to(DEV) for x in (a8, as_, w8, ws)), out_i32=c)
    torch.cuda.synchronize()
    c_ref = orc.gemm_i32(a8, w8, threads=8)
    assert np.array_equal(c.cpu().numpy(), c_ref)
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(orc.rescale(c_ref, as_, ws)))


def _gemv_cases(count=30, seed=7):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        kind = int(g.choice([4, 6]))
        k = 256 * int(g.integers(1, 41))
        m = int(g.choice([1, 1, 2, 3, 4, 4, int(g.integers(5, 17))]))
        ns = tuple(int(g.integers(1, 1500)) for _ in range(int(g.integers(1, 4))))
        out.append((kind, ns, k, m))
    return out


@pytest.mark.parametrize("kind,ns,k,m", _gemv_cases())
def test_fused_gemv_random_shape(kind, ns, k, m):
    print(f"random gemv kind={kind} ns={ns} k={k} m={m}", flush=True)
    ws = [synth.kquant(kind, n, k, index=9000 + i * 17 + n) for i, n in enumerate(ns)]
    x = synth.activations(m, k, index=9100 + m + k)
    outs = hip.gemv_q_f32(kind, [torch.from_numpy(w).to(DEV) for w in ws], k, ns, torch.from_numpy(x).to(DEV))
    torch.cuda.synchronize()
    q8 = orc.quantize_q8_k(x)
    for w, n, o in zip(ws, ns, outs):
        got = o.cpu().numpy()
        ref = orc.gemv_q8_k(kind, w, k, n, q8, threads=8)
        for mi in range(m):
            _, _, mag = orc.gemv_block_sums(kind, w, k, n, q8[mi])
            err = np.abs(got[mi].astype(np.float64) - ref[mi])
            assert np.all(err <= 1e-5 * mag), f"member n={n} row {mi}: max err/mag {np.max(err / mag)}"
            assert err.max() <= 1e-5 * np.abs(ref[mi]).max(), "normwise max|err| / max|y|"


def _capi_cases(count=24, seed=99):
    g = np.random.default_rng(seed)
    out = []
    for i in range(count):
        kind = int(g.choice([4, 5, 6]))
        m = int(g.choice([1, int(g.integers(2, 17)), int(g.integers(17, 300))]))
        if kind == 5 and m == 1:
            m = 2  # the reference rejects Q5_K at one row
        k = 256 * int(g.integers(1, 25))
        # the grouped entry takes Q4_K and Q6_K only, as the reference's (lib.rs:2573-2577)
        ns = tuple(int(g.integers(1, 2500)) for _ in range(1 if kind == 5 else int(g.integers(1, 4))))
        out.append((kind, m, k, ns))
    return out


@pytest.mark.parametrize("kind,m,k,ns", _capi_cases())
def test_capi_random_shape_bit_exact(kind, m, k, ns):
    """The reference C ABI on host buffers (rocknpu_matmul_q{4,5,6}_k_f32_f32 for one
    projection, rocknpu_matmul_q_concat_f32_f32_mtile for several sharing the
    activations): the W8A8 route, bit for bit against the oracle."""
    from rocknpu_amd.capi import STATUS_OK, Context

    print(f"random capi kind={kind} m={m} k={k} ns={ns}", flush=True)
    ws = [synth.kquant(kind, n, k, index=9500 + i * 13 + n) for i, n in enumerate(ns)]
    a = synth.activations(m, k, index=9600 + m + k)
    with Context() as ctx:
        if len(ns) == 1:
            out = np.empty((m, ns[0]), np.float32)
            assert ctx.matmul_q(kind, ws[0], a, out, k, ns[0]) == STATUS_OK
            outs = [out]
        else:
            outs = [np.empty((m, n), np.float32) for n in ns]
            assert ctx.matmul_q_concat(ws, [kind] * len(ns), list(ns), a, outs, k) == STATUS_OK
        for w, n, o in zip(ws, ns, outs):
            assert np.array_equal(_bits(o), _bits(orc.matmul_q_w8a8(kind, w, a, n, threads=8))), f"member n={n}"
