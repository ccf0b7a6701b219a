"""rocknpu_hip_matmul_w8a8_f32_noalloc (fixed per-GPU workspace, no allocation)
against rocknpu_hip_matmul_w8a8_f32 (library-allocated workspace), through the
C ABI: bit-identical outputs on two calls in a row, the second smaller (the
workspace keeps the first call's bytes), and the size limit."""
import ctypes

import numpy as np
import pytest
import torch

from rocknpu_amd import _lib, hip, synth

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _call(fn, a, k, w8, ws, out):
    m, lda = a.shape[0], a.stride(0)
    n, k_pad = w8.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return fn(_p(a), m, k, lda, _p(w8), _p(ws), n, k_pad, _p(out), out.stride(0), stream)


def test_noalloc_equals_allocating_entry_point_twice():
    lib = _lib.load()
    for kind, m, k, n, lda in ((4, 300, 5632, 2048, 5632), (6, 17, 2048, 640, 2056)):
        print(f"noalloc kind={kind} m={m} k={k} n={n}", flush=True)
        blocks = synth.kquant(kind, n, k, index=3000 + m)
        a = torch.from_numpy(synth.activations(m, lda, index=3001 + m)).to("cuda")
        w8, ws = hip.repack_w8(kind, torch.from_numpy(blocks).to("cuda"), k, n)
        ref = torch.full((m, n), float("nan"), device="cuda")
        got = torch.full((m, n), float("nan"), device="cuda")
        assert _call(lib.rocknpu_hip_matmul_w8a8_f32, a, k, w8, ws, ref) == 0
        assert _call(lib.rocknpu_hip_matmul_w8a8_f32_noalloc, a, k, w8, ws, got) == 0
        torch.cuda.synchronize()
        r, g = ref.cpu().numpy(), got.cpu().numpy()
        assert np.isfinite(r).all()
        assert np.array_equal(r.view(np.uint32), g.view(np.uint32))


def test_noalloc_rejects_sizes_beyond_its_workspace():
    lib = _lib.load()
    a = torch.zeros((16385, 64), device="cuda")
    w8 = torch.zeros((64, 64), dtype=torch.int8, device="cuda")
    ws = torch.ones(64, device="cuda")
    out = torch.zeros((16385, 64), device="cuda")
    assert _call(lib.rocknpu_hip_matmul_w8a8_f32_noalloc, a, 64, w8, ws, out) == -1   # rows
    a2 = torch.zeros((512, 65600), device="cuda")
    w2 = torch.zeros((8, 65600), dtype=torch.int8, device="cuda")
    o2 = torch.zeros((512, 8), device="cuda")
    assert 512 * 65600 > 32 << 20
    assert _call(lib.rocknpu_hip_matmul_w8a8_f32_noalloc, a2, 65600, w2, ws, o2) == -1  # bytes
