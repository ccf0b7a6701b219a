"""The HIP kernels reproduce the golden fixtures (tests/golden): bit-exact for
the int8/i32 intermediates and the rescaled f32 GEMM output, and within
1e-5 of the row's block magnitude for the decode GEMV's f32 accumulation."""
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLD / f"{name}.npz", allow_pickle=False)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def test_gpu_golden_quantize_a8():
    import torch
    from rocknpu_amd import hip
    for name in ("rounding_kat", "max_abs_kat"):
        f = _load(name)
        a8, sc = hip.quantize_a8(_dev(f["x"][None]), len(f["x"]) + (-len(f["x"]) % 64))
        torch.cuda.synchronize()
        assert np.array_equal(a8.cpu().numpy()[0, :len(f["x"])], f["q"]), name
        assert _bits(sc.cpu().numpy())[0] == _bits(f["scale"])[0], name
    f = _load("quantize_a8")
    a8, sc = hip.quantize_a8(_dev(f["a"]), int(f["k_pad"]))
    torch.cuda.synchronize()
    assert np.array_equal(a8.cpu().numpy(), f["a8"]) and np.array_equal(_bits(sc.cpu().numpy()), _bits(f["scales"]))


def test_gpu_golden_gemm_kats():
    import torch
    from rocknpu_amd import hip
    f = _load("gemm_kats")
    for name in ("m1", "m1_neg", "mtile_uniform", "ksplit"):
        print(f"golden gemm {name}", flush=True)
        a, w = f[f"{name}_a"], f[f"{name}_w"]
        c = torch.empty((a.shape[0], w.shape[0]), dtype=torch.int32, device="cuda")
        out = hip.gemm_w8a8(_dev(a), _dev(f[f"{name}_as"]), _dev(w), _dev(f[f"{name}_ws"]), out_i32=c)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), f[f"{name}_c"]), name
        assert np.array_equal(_bits(out.cpu().numpy()), _bits(f[f"{name}_out"])), name


@pytest.mark.parametrize("kind", [4, 6])
def test_gpu_golden_repack(kind):
    import torch
    from rocknpu_amd import hip
    f = _load(f"repack_q{kind}k")
    w8, sc = hip.repack_w8(kind, _dev(f["blocks"]), int(f["k"]), int(f["n"]))
    torch.cuda.synchronize()
    assert np.array_equal(w8.cpu().numpy(), f["w8"]) and np.array_equal(_bits(sc.cpu().numpy()), _bits(f["scales"]))


def test_gpu_golden_q8_k():
    import torch
    from rocknpu_amd import hip
    f = _load("q8_k")
    q = hip.quantize_q8_k(_dev(f["x"]))
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), f["q8k"])


@pytest.mark.parametrize("kind", [4, 6])
def test_gpu_golden_gemv(kind):
    import torch
    from rocknpu_amd import hip
    f = _load(f"gemv_q{kind}k")
    k, n = int(f["k"]), int(f["n"])
    m, nb = f["q8k"].shape[0], k // 256
    isum = torch.empty((m, n, nb), dtype=torch.int32, device="cuda")
    msum = torch.empty((m, n, nb), dtype=torch.int32, device="cuda")
    out = hip.gemv_q8_k(kind, _dev(f["w"]), k, n, _dev(f["q8k"]), isum=isum, msum=msum)
    fused = hip.gemv_q_f32(kind, [_dev(f["w"])], k, [n], _dev(f["x"]))[0]
    torch.cuda.synchronize()
    assert np.array_equal(isum.cpu().numpy(), f["isum"]) and np.array_equal(msum.cpu().numpy(), f["msum"])
    for got in (out.cpu().numpy(), fused.cpu().numpy()):
        assert np.all(np.abs(got.astype(np.float64) - f["y"]) <= 1e-5 * f["mag"] + 1e-30)


def test_gpu_golden_q5_k_high_bits():
    """The Q5_K repack kernel on single-bit blocks: W8 and scales equal the
    closed form's quantisation bit for bit."""
    import torch
    from rocknpu_amd import hip
    f = _load("repack_q5k_bits")
    w8, sc = hip.repack_w8(5, _dev(f["blocks"]), 256, int(f["n"]))
    torch.cuda.synchronize()
    assert np.array_equal(w8.cpu().numpy(), f["w8"]) and np.array_equal(_bits(sc.cpu().numpy()), _bits(f["scales"]))


@pytest.mark.parametrize("kind", [4, 6])
def test_gpu_golden_q8_k_half_even_ties(kind):
    """Exact ties of iscale * x round half to even on the GPU: the Q8_K
    quantiser reproduces the fixture, and the GEMV that quantises in-kernel
    equals the GEMV on those Q8_K bytes bit for bit (so it rounds the same)."""
    import torch
    from rocknpu_amd import hip, synth
    f = _load("q8_k_ties")
    q = hip.quantize_q8_k(_dev(f["x"]))
    torch.cuda.synchronize()
    q = q.cpu().numpy()
    assert np.array_equal(q[0, :292], f["q8k_block0"])
    n, k = 48, 512
    w = _dev(synth.kquant(kind, n, k, index=960 + kind))
    for m in (1, 4):
        x = np.repeat(f["x"], m, axis=0)
        x[1:] *= np.float32(0.5)  # further rows: ties at the half-scale grid
        q8 = hip.quantize_q8_k(_dev(x))
        ref = hip.gemv_q8_k(kind, w, k, n, q8)
        fused = hip.gemv_q_f32(kind, [w], k, [n], _dev(x))[0]
        torch.cuda.synchronize()
        assert np.array_equal(_bits(fused.cpu().numpy()), _bits(ref.cpu().numpy())), m
