"""Column-split W8A8 GEMM on the GPU (launch_gemm_w8a8, include/rocknpu_hip.h
rocknpu_hip_gemm_column_split): a product whose 256 x 256 tiles make whole
rounds plus a last round at most half full runs as two launches (the whole
rounds' columns on 256 x 256 tiles, the rest routed on its own). Its int32
accumulators and f32 outputs are those of one 256 x 256 launch over the
whole product bit for bit, and its int32 accumulators are the exact products
(numpy int64) on sampled rows; the same through the C ABI's device prompt
route, and in graph replays."""
import ctypes

import numpy as np
import pytest
import torch

from rocknpu_amd import _lib, hip

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _n0(m, n, k):
    n0 = ctypes.c_size_t()
    assert _lib.load().rocknpu_hip_gemm_column_split(m, n, k, 0, ctypes.byref(n0)) == 0
    return n0.value


def _operands(m, n, k, seed):
    g = np.random.default_rng(seed)
    a8 = g.integers(-127, 128, (m, k), dtype=np.int8)
    w8 = g.integers(-127, 128, (n, k), dtype=np.int8)
    as_ = (g.random(m, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    ws = (g.random(n, dtype=np.float32) + np.float32(0.01)) / np.float32(127)
    return a8, w8, as_, ws


@pytest.mark.parametrize("m,n,k", [
    (1536, 11264, 2048),   # one round + 8 tiles
    (768, 28672, 1024),    # one round + 80
    (4096, 5632, 1024),    # one round + 96
    (1300, 11000, 640),    # ragged M and N: 6 x 43 = 258 tiles, a 248-column tail
])
def test_column_split_equals_one_launch(m, n, k):
    n0 = _n0(m, n, k)
    assert n0 > 0, (m, n, k, torch.cuda.get_device_properties(0).multi_processor_count)
    print(f"column split m={m} n={n} k={k} n0={n0}", flush=True)
    a8, w8, as_, ws = _operands(m, n, k, seed=m + n + k)
    a8d, w8d = torch.from_numpy(a8).to(DEV), torch.from_numpy(w8).to(DEV)
    asd, wsd = torch.from_numpy(as_).to(DEV), torch.from_numpy(ws).to(DEV)
    i32 = torch.empty((m, n), dtype=torch.int32, device=DEV)
    out = hip.gemm_w8a8(a8d, asd, w8d, wsd, out_i32=i32)
    i32_one = torch.empty_like(i32)
    one = hip.gemm_w8a8_tile(256, 256, 2, 1, a8d, asd, w8d, wsd, out_i32=i32_one)
    torch.cuda.synchronize()
    assert torch.equal(i32, i32_one)
    assert torch.equal(out.view(torch.int32), one.view(torch.int32))
    # exact products on rows at both ends and in the middle, every column
    rows = [0, 1, m // 2, m - 2, m - 1]
    want = a8[rows].astype(np.int64) @ w8.astype(np.int64).T
    assert np.array_equal(i32[rows].cpu().numpy().astype(np.int64), want)
    # the rescale of those rows: (f32(acc) * a_scale) * w_scale
    got = out[rows].cpu().numpy()
    ref = (want.astype(np.float32) * as_[rows, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_column_split_graph_replays_match_eager():
    m, n, k = 1536, 11264, 1024
    assert _n0(m, n, k) > 0
    a8, w8, as_, ws = _operands(m, n, k, seed=7)
    a8d, w8d = torch.from_numpy(a8).to(DEV), torch.from_numpy(w8).to(DEV)
    asd, wsd = torch.from_numpy(as_).to(DEV), torch.from_numpy(ws).to(DEV)
    eager = hip.gemm_w8a8(a8d, asd, w8d, wsd)
    out = torch.zeros_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hip.gemm_w8a8(a8d, asd, w8d, wsd, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        hip.gemm_w8a8(a8d, asd, w8d, wsd, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
