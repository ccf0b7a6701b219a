"""Device-tensor wrappers of the launch layer (include/rocknpu_hip.h).

Arguments are torch tensors already resident on the GPU; calls enqueue on the
current torch stream and return immediately. torch is used only for device
memory and streams; the computation is the gfx950 kernels of the library.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

QK = 256
Q8K_BYTES = 292
BLOCK_BYTES = {4: 144, 5: 176, 6: 210}


class LaunchError(RuntimeError):
    pass


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check(status: int, what: str) -> None:
    if status != 0:
        raise LaunchError(f"{what} returned status {status}")


def _ld(t: torch.Tensor) -> int:
    """Row stride in elements for the C ABI. A single row's stride is
    arbitrary in torch (0 for a row added with [None]), so it is the row
    length there."""
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def k_pad_of(k: int) -> int:
    return (k + 63) // 64 * 64


def repack_w8(kind: int, blocks: torch.Tensor, k: int, n: int, w8: torch.Tensor | None = None,
              scales: torch.Tensor | None = None):
    """Kernel (a): K-quant blocks -> (W8 [n, k_pad] int8, scales [n] f32)."""
    kp = k_pad_of(k)
    if w8 is None:
        w8 = torch.empty((n, kp), dtype=torch.int8, device=blocks.device)
    if scales is None:
        scales = torch.empty(n, dtype=torch.float32, device=blocks.device)
    assert w8.shape == (n, kp) and w8.is_contiguous() and scales.numel() == n
    _check(_lib.load().rocknpu_hip_repack_w8(kind, _ptr(blocks), blocks.numel(), k, n, kp, _ptr(w8),
                                             _ptr(scales), _stream()), "repack_w8")
    return w8, scales


def quantize_a8(a: torch.Tensor, k_pad: int | None = None, a8: torch.Tensor | None = None,
                scales: torch.Tensor | None = None):
    """Kernel (b): f32 [m, k] -> (A8 [m, k_pad] int8, scales [m] f32)."""
    m, k = a.shape
    kp = k_pad_of(k) if k_pad is None else k_pad
    if a8 is None:
        a8 = torch.empty((m, kp), dtype=torch.int8, device=a.device)
    if scales is None:
        scales = torch.empty(m, dtype=torch.float32, device=a.device)
    _check(_lib.load().rocknpu_hip_quantize_a8(_ptr(a), m, k, _ld(a), kp, _ptr(a8), _ptr(scales),
                                               _stream()), "quantize_a8")
    return a8, scales


def gemm_workspace(m: int, n: int, k_pad: int, cus: int = 0) -> tuple[int, int]:
    """(bytes, K splits) of the workspace the GEMM's route uses for m x n x k_pad."""
    nb = ctypes.c_size_t()
    sp = ctypes.c_int()
    _check(_lib.load().rocknpu_hip_gemm_workspace(m, n, k_pad, cus, ctypes.byref(nb), ctypes.byref(sp)),
           "gemm_workspace")
    return nb.value, sp.value


def gemm_column_split(m: int, n: int, k_pad: int, cus: int = 0) -> int:
    """Columns of the first of the two launches the GEMM runs an m x n x k_pad
    product as (0: one launch); rocknpu_hip_gemm_column_split."""
    n0 = ctypes.c_size_t()
    _check(_lib.load().rocknpu_hip_gemm_column_split(m, n, k_pad, cus, ctypes.byref(n0)), "gemm_column_split")
    return n0.value


# Zeroed K-split workspaces, one per (device, stream): the GEMM leaves them
# zeroed, so each is zeroed once, when it is made. Calls on one stream are
# ordered with each other, so they can share its workspace; calls on other
# streams get their own. Under HIP graph capture none is made or grown (the
# zeroing would run only at replay, and eager calls would find the counters
# dirty); a captured call runs unsplit unless the stream already has a large
# enough workspace, which the graph then reuses on every replay.
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def workspace_for(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """This module's zeroed workspace of at least nbytes for the current
    stream on `device`; None when one would have to be made or grown during
    graph capture."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(index)
    key = (index, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        return None
    new = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", index))
    if ws is not None:
        # the old buffer may still be read by work queued on this stream
        ws.record_stream(stream)
    _workspaces[key] = new
    return new


def gemm_workspace_check(workspace: torch.Tensor) -> bool:
    """Waits for the current stream and reads and clears the workspace's error
    word: True when no split GEMM on it found dirty counters since the last
    check. A False workspace must be zeroed before it is used again."""
    st = _lib.load().rocknpu_hip_gemm_workspace_check(_ptr(workspace), _stream())
    if st not in (0, -3):
        raise LaunchError(f"gemm_workspace_check returned status {st}")
    return st == 0


def gemm_w8a8(a8: torch.Tensor, a_scales: torch.Tensor, w8: torch.Tensor, w_scales: torch.Tensor,
              out: torch.Tensor | None = None, out_i32: torch.Tensor | None = None,
              workspace: torch.Tensor | bool | None = True) -> torch.Tensor:
    """Kernel (c): out[m, n] = (f32(A8 W8^T) * a_scales) * w_scales.

    workspace: True (default) splits K where the route does, in this module's
    zeroed workspace for the current stream (none under graph capture unless
    the stream already has one; the call then runs unsplit); a uint8 device
    tensor supplies one (zeroed once by the caller, used by one stream at a
    time); None or False runs the call without one (rocknpu_hip_gemm_w8a8,
    never split). The bits are the same either way."""
    m, kp = a8.shape
    n = w8.shape[0]
    assert w8.shape[1] == kp and a8.is_contiguous() and w8.is_contiguous()
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a8.device)
    lib = _lib.load()
    if workspace is True:
        nbytes, _ = gemm_workspace(m, n, kp)
        workspace = workspace_for(a8.device, nbytes) if nbytes else None
    if workspace is None or workspace is False:
        _check(lib.rocknpu_hip_gemm_w8a8(_ptr(a8), _ptr(a_scales), _ptr(w8), _ptr(w_scales), m, n, kp,
                                         _ptr(out), _ld(out), _ptr(out_i32), _stream()), "gemm_w8a8")
        return out
    _check(lib.rocknpu_hip_gemm_w8a8_ws(_ptr(a8), _ptr(a_scales), _ptr(w8), _ptr(w_scales), m, n, kp, _ptr(out),
                                        _ld(out), _ptr(out_i32), _ptr(workspace), workspace.numel(), _stream()),
           "gemm_w8a8_ws")
    return out


def gemm_w8a8_tile(bm: int, bn: int, stages: int, splits: int, a8: torch.Tensor, a_scales: torch.Tensor,
                   w8: torch.Tensor, w_scales: torch.Tensor, out: torch.Tensor | None = None,
                   out_i32: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Kernel (c) on a given tile, stage count and K split (tests and tuning)."""
    m, kp = a8.shape
    n = w8.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a8.device)
    _check(_lib.load().rocknpu_hip_gemm_w8a8_tile(bm, bn, stages, splits, _ptr(a8), _ptr(a_scales), _ptr(w8),
                                                  _ptr(w_scales), m, n, kp, _ptr(out), _ld(out), _ptr(out_i32),
                                                  _ptr(workspace), 0 if workspace is None else workspace.numel(),
                                                  _stream()), "gemm_w8a8_tile")
    return out


def matmul_w8a8_f32(a: torch.Tensor, w8: torch.Tensor, w_scales: torch.Tensor, k: int | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Kernels (b) + (c) in one call: f32 activations a [m, >= k] quantised per
    token into a library workspace, times the resident W8 [n, k_pad]."""
    m = a.shape[0]
    k = a.shape[1] if k is None else k
    n, kp = w8.shape
    assert w8.is_contiguous() and a.stride(1) == 1
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    _check(_lib.load().rocknpu_hip_matmul_w8a8_f32(_ptr(a), m, k, _ld(a), _ptr(w8), _ptr(w_scales), n, kp,
                                                   _ptr(out), _ld(out), _stream()), "matmul_w8a8_f32")
    return out


def quantize_q8_k(x: torch.Tensor, q8k: torch.Tensor | None = None) -> torch.Tensor:
    """f32 [m, k] -> Q8_K rows, uint8 [m, (k/256)*292]."""
    m, k = x.shape
    if q8k is None:
        q8k = torch.empty((m, (k // QK) * Q8K_BYTES), dtype=torch.uint8, device=x.device)
    _check(_lib.load().rocknpu_hip_quantize_q8_k(_ptr(x), m, k, _ld(x), _ptr(q8k), _stream()),
           "quantize_q8_k")
    return q8k


def gemv_q8_k(kind: int, w: torch.Tensor, k: int, n: int, q8k: torch.Tensor, out: torch.Tensor | None = None,
              isum: torch.Tensor | None = None, msum: torch.Tensor | None = None) -> torch.Tensor:
    """Kernel (d): out[m, n] = vec_dot(W row, Q8_K row) for Q4_K / Q6_K weights."""
    m = q8k.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=q8k.device)
    _check(_lib.load().rocknpu_hip_gemv_q8_k(kind, _ptr(w), w.numel(), k, n, _ptr(q8k), m, _ptr(out),
                                             _ld(out), _ptr(isum), _ptr(msum), _stream()), "gemv_q8_k")
    return out


def gemv_q_f32(kind: int, weights, k: int, ns, x: torch.Tensor, outs=None):
    """Kernel (d), fused: f32 activations x [m, k] quantised to Q8_K in-kernel,
    times 1..4 same-kind projections sharing x. Returns the list of outputs."""
    m = x.shape[0]
    count = len(weights)
    if outs is None:
        outs = [torch.empty((m, n), dtype=torch.float32, device=x.device) for n in ns]
    w_arr = (ctypes.c_void_p * count)(*[w.data_ptr() for w in weights])
    b_arr = (ctypes.c_size_t * count)(*[w.numel() for w in weights])
    n_arr = (ctypes.c_size_t * count)(*ns)
    o_arr = (ctypes.c_void_p * count)(*[o.data_ptr() for o in outs])
    l_arr = (ctypes.c_size_t * count)(*[_ld(o) for o in outs])
    _check(_lib.load().rocknpu_hip_gemv_q_f32(kind, count, w_arr, b_arr, n_arr, k, _ptr(x), _ld(x), m,
                                              o_arr, l_arr, _stream()), "gemv_q_f32")
    return outs


def gemv_tiled_bytes(kind: int, k: int, n: int) -> int:
    """Bytes of the tile-interleaved decode copy of an n x k Q4_K/Q6_K weight."""
    nb = _lib.load().rocknpu_hip_gemv_tiled_bytes(kind, k, n)
    if nb == 0:
        raise LaunchError(f"gemv_tiled_bytes: invalid kind {kind} or shape {n} x {k}")
    return nb


def gemv_tile_weights(kind: int, w: torch.Tensor, k: int, n: int, tiled: torch.Tensor | None = None) -> torch.Tensor:
    """Raw GGUF blocks [n rows of k/256 blocks] -> their tile-interleaved copy
    (uint8, gemv_tiled_bytes long) for the tiled decode GEMV."""
    nbytes = gemv_tiled_bytes(kind, k, n)
    if tiled is None:
        tiled = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _check(_lib.load().rocknpu_hip_gemv_tile_weights(kind, _ptr(w), w.numel(), k, n, _ptr(tiled), tiled.numel(),
                                                     _stream()), "gemv_tile_weights")
    return tiled


def gemv_tiled_workspace_bytes(kind: int, m: int, k: int, rows: int) -> int:
    """Bytes of the K-split workspace a tiled GEMV call of m rows over K = k
    and `rows` output rows in all needs (0: none of its launches splits)."""
    return int(_lib.load().rocknpu_hip_gemv_tiled_workspace_bytes(kind, m, k, rows))


# The tiled GEMV's K-split workspaces, one per (device, stream), each zeroed
# when made; every completed call leaves its workspace zero. Under graph
# capture none is made or grown (the zeroing would run only at replay): a
# captured split call needs the stream to have one already, from an eager call
# on it, and raises otherwise.
_gemv_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def gemv_workspace_for(device: torch.device, nbytes: int) -> torch.Tensor:
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(index)
    key = (index, stream.cuda_stream)
    ws = _gemv_workspaces.get(key)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        raise LaunchError("a split tiled GEMV under graph capture needs this stream's K-split workspace: "
                          "make one eager call of the same shape on the capturing stream first")
    new = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=torch.device("cuda", index))
    if ws is not None:
        ws.record_stream(stream)
    _gemv_workspaces[key] = new
    return new


def gemv_workspace_check(workspace: torch.Tensor) -> bool:
    """Waits for the current stream and reads and clears the tiled GEMV
    workspace's error word: True when no split call on it found it not clear
    since the last check. A False workspace must be zeroed before reuse."""
    st = _lib.load().rocknpu_hip_gemv_tiled_workspace_check(_ptr(workspace), _stream())
    if st not in (0, -3):
        raise LaunchError(f"gemv_tiled_workspace_check returned status {st}")
    return st == 0


def _gemv_ws(kind: int, m: int, k: int, rows: int, device, workspace):
    need = gemv_tiled_workspace_bytes(kind, m, k, rows)
    if need == 0:
        return None, 0
    ws = gemv_workspace_for(device, need) if workspace is None else workspace
    return ws, ws.numel()


def gemv_q_f32_tiled(kind: int, weights, k: int, ns, x: torch.Tensor, outs=None,
                     workspace: torch.Tensor | None = None):
    """gemv_q_f32 on tiled copies (gemv_tile_weights) of 1..4 projections.
    Split launches (rows of 17-31 blocks at 2-8 activation rows) use
    `workspace`, or this stream's own (gemv_workspace_for)."""
    m = x.shape[0]
    count = len(weights)
    if outs is None:
        outs = [torch.empty((m, n), dtype=torch.float32, device=x.device) for n in ns]
    ws, ws_bytes = _gemv_ws(kind, m, k, sum(ns), x.device, workspace)
    w_arr = (ctypes.c_void_p * count)(*[w.data_ptr() for w in weights])
    b_arr = (ctypes.c_size_t * count)(*[w.numel() for w in weights])
    n_arr = (ctypes.c_size_t * count)(*ns)
    o_arr = (ctypes.c_void_p * count)(*[o.data_ptr() for o in outs])
    l_arr = (ctypes.c_size_t * count)(*[_ld(o) for o in outs])
    _check(_lib.load().rocknpu_hip_gemv_q_f32_tiled(kind, count, w_arr, b_arr, n_arr, k, _ptr(x), _ld(x), m,
                                                    o_arr, l_arr, _ptr(ws), ws_bytes, _stream()), "gemv_q_f32_tiled")
    return outs


def gemv_q8_k_tiled(kind: int, w: torch.Tensor, k: int, n: int, q8k: torch.Tensor,
                    out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """gemv_q8_k on a tiled copy (gemv_tile_weights); split launches as in
    gemv_q_f32_tiled."""
    m = q8k.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=q8k.device)
    ws, ws_bytes = _gemv_ws(kind, m, k, n, q8k.device, workspace)
    _check(_lib.load().rocknpu_hip_gemv_q8_k_tiled(kind, _ptr(w), w.numel(), k, n, _ptr(q8k), m, _ptr(out),
                                                   _ld(out), _ptr(ws), ws_bytes, _stream()), "gemv_q8_k_tiled")
    return out


def gemv_tiled_preferred(kind: int, m: int, k: int) -> bool:
    """Whether an m-row decode GEMV over K = k runs faster on the tiled copy
    than on raw rows: from two rows, and at one row for rows of 5-20, 25-27
    and 32 or more blocks (Q6_K: up to 64)."""
    return bool(_lib.load().rocknpu_hip_gemv_tiled_preferred(kind, m, k))


def gemv_decode(kind: int, raw, tiled, k: int, ns, x: torch.Tensor, outs=None):
    """The fused decode GEMV on whichever copy gemv_tiled_preferred picks:
    `raw` and `tiled` are the members' raw GGUF rows and their tiled copies
    (either list may be None when the rule never picks it for this call)."""
    if gemv_tiled_preferred(kind, x.shape[0], k):
        return gemv_q_f32_tiled(kind, tiled, k, ns, x, outs=outs)
    return gemv_q_f32(kind, raw, k, ns, x, outs=outs)


def gemv_take_stall() -> bool:
    """Whether a GEMV launch with a bounded wait for the activations (the fused
    lane-per-block kernel, the Q6_K stream kernel) gave up since the last call
    (call after synchronising); clears the flag."""
    return bool(_lib.load().rocknpu_hip_gemv_take_stall())


def gemv_test_stall(spins: int) -> None:
    """Test hook: spins > 0 makes later launches with that wait wait for an
    arrival that never comes and give up after `spins` polls; 0 restores."""
    _check(_lib.load().rocknpu_hip_gemv_test_stall(spins), "gemv_test_stall")
