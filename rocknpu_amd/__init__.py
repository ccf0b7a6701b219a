"""MI355X (gfx950) implementation of RockNPU's ggml MUL_MAT offload path.

Layers:
  include/rocknpu.h        the reference's C ABI (drop-in, host pointers)
  include/rocknpu_ggml.h   decode MUL_MAT with llama.cpp CPU numerics
  include/rocknpu_hip.h    device-pointer launch layer of the four kernels
  rocknpu_amd.capi         numpy mirror of rocknpu.h
  rocknpu_amd.hip          torch-device wrappers of rocknpu_hip.h
  rocknpu_amd.synth        deterministic synthetic GGUF weights / activations
"""
from . import _lib, synth  # noqa: F401

LIB_PATH = _lib.LIB_PATH


def load():
    """Load librocknpu_capi.so; raises ImportError when it has not been built."""
    return _lib.load()
