"""The W8 sidecar (include/rocknpu_sidecar.h) from Python: repacked int8
weights cached on disk with a provenance fingerprint of their GGUF source.

Mirrors the reference's generator (scripts/make_tinyllama_w8_sidecar_gguf.py:
46-70 quantize_rows, 101-158 the per-tensor files and manifest.json) and its
reader (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:209-259), with the
conversion done by the GPU repack (round half away from zero, the plugin's
rocknpu_w8_convert semantics; the generator script rounds with floor(x+0.5),
which differs at exact .5 ties of negative values).
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

from . import _lib

FORMAT = "rocknpu-w8-sidecar-v2"
GGML_TYPE = {4: 12, 5: 13, 6: 14}  # ggml_type ids of Q4_K, Q5_K, Q6_K


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def fingerprint(source: np.ndarray) -> int:
    """FNV-1a 64 of the byte count and sampled bytes of a GGUF source tensor."""
    src = np.ascontiguousarray(source).view(np.uint8).reshape(-1)
    return int(_lib.load().rocknpu_w8_source_fingerprint(_p(src), src.nbytes))


def write(directory, name: str, source: np.ndarray, w8: np.ndarray, scales: np.ndarray) -> int:
    src = np.ascontiguousarray(source).view(np.uint8).reshape(-1)
    w8 = np.ascontiguousarray(w8, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    n, k = w8.shape
    return _lib.load().rocknpu_w8_sidecar_write(str(directory).encode(), name.encode(), _p(src), src.nbytes, k, n,
                                                _p(w8), _p(scales))


def read(directory, name: str, source: np.ndarray, k: int, n: int):
    """(w8 [n, k], scales [n]) when the sidecar matches the source, else None."""
    src = np.ascontiguousarray(source).view(np.uint8).reshape(-1)
    w8 = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    st = _lib.load().rocknpu_w8_sidecar_read(str(directory).encode(), name.encode(), _p(src), src.nbytes, k, n,
                                             _p(w8), _p(sc))
    return (w8, sc) if st == 0 else None


def get(context, directory, name: str, kind: int, source: np.ndarray, k: int, n: int, write_back: bool = False):
    """(status, w8, scales, from_sidecar): the sidecar when it matches, else the GPU
    repack of the K-quant source (written back as a sidecar when asked)."""
    src = np.ascontiguousarray(source).view(np.uint8).reshape(-1)
    w8 = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    hit = ctypes.c_int(0)
    d = None if directory is None else str(directory).encode()
    st = _lib.load().rocknpu_w8_sidecar_get(context.handle, d, name.encode(), kind, _p(src), src.nbytes, k, n,
                                            _p(w8), _p(sc), 1 if write_back else 0, ctypes.byref(hit))
    return st, w8, sc, bool(hit.value)


def make_directory(context, directory, tensors, source_desc: str = "") -> dict:
    """Write sidecars for {name: (kind, blocks, k, n)} and the generator's
    manifest.json (make_tinyllama_w8_sidecar_gguf.py:101-158)."""
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    manifest = {"format": FORMAT, "source": source_desc,
                "source_semantics": "GGUF tensor dequantize -> symmetric-per-output-channel-int8",
                "rounding": "half-away-from-zero", "tensors": {}}
    for name, (kind, blocks, k, n) in tensors.items():
        st, _, _, _ = get(context, out, name, kind, blocks, k, n, write_back=True)
        if st != 0:
            raise RuntimeError(f"{name}: sidecar conversion failed with status {st}")
        manifest["tensors"][name] = {"k": k, "n": n, "scheme": "symmetric-per-output-channel-int8",
                                     "ggml_type": GGML_TYPE[kind],
                                     "source_sample_fnv1a64": f"{fingerprint(blocks):016x}"}
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest
