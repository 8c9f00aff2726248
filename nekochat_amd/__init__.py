"""nekochat_amd: MI355X (gfx950) kernels for NekoChat's per-row transformer layer ops.

LayerNorm, RMSNorm (incl. Qwen3 q/k head norm and Granite's gated group norm), GELU-tanh, SwiGLU,
NeoX RoPE and the embedding gather with FP16/FP8/FP4 row dequantisation, as hand-written HIP kernels
behind the C ABI in include/neko_hip.h (libneko_hip.so, built in-tree). The C++ ComputeBackend
adapter (csrc/hip_backend.cpp) keeps the reference engine's per-op backend interface; `ops` is the
torch-facing mirror of the same interface.
"""
from ._lib import LIB_PATH, NekoError  # noqa: F401  (raises ImportError if the library is not built)
from . import ops  # noqa: F401

__all__ = ["ops", "NekoError", "LIB_PATH"]
