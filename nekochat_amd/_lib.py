"""ctypes binding to libneko_hip.so, the C ABI declared in include/neko_hip.h.

The library is built in-tree (nekochat_amd/libneko_hip.so). If it is missing this module raises at
import: there is no CPU fallback for any op.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libneko_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "neko_hip.h")

NEKO_OK = 0
NEKO_ERR_INVALID = -1
NEKO_ERR_HIP = -2
NEKO_ERR_NO_DEVICE = -3
NEKO_ERR_UNSUPPORTED = -4

DT_F32, DT_F16 = 0, 1
FMT_F16, FMT_FP8, FMT_FP4 = 0, 1, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the order of include/neko_hip.h.
SIGNATURES = {
    "neko_hip_create": (_i32, [_i32, ctypes.POINTER(_p)]),
    "neko_hip_destroy": (_i32, [_p]),
    "neko_hip_last_error": (ctypes.c_char_p, [_p]),
    "neko_hip_device_name": (_i32, [_p, ctypes.c_char_p, _sz]),
    "neko_hip_max_buffer_bytes": (_sz, [_p]),
    "neko_hip_set_stream": (_i32, [_p, _p]),
    "neko_hip_get_stream": (_p, [_p]),
    "neko_hip_alloc": (_i32, [_p, _sz, ctypes.POINTER(_p)]),
    "neko_hip_free": (_i32, [_p, _p]),
    "neko_hip_upload": (_i32, [_p, _p, _p, _sz]),
    "neko_hip_download": (_i32, [_p, _p, _p, _sz]),
    "neko_hip_memset": (_i32, [_p, _p, _i32, _sz]),
    "neko_hip_synchronize": (_i32, [_p]),
    "neko_hip_layernorm": (_i32, [_p, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _f32, _i32]),
    "neko_hip_rmsnorm": (_i32, [_p, _p, _i64, _p, _i64, _p, _i64, _i64, _f32, _i32]),
    "neko_hip_gated_rmsnorm": (_i32, [_p, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i32, _f32, _i32]),
    "neko_hip_qk_norm_rope": (_i32, [_p, _p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32, _i32]),
    "neko_hip_qk_norm_rope_kv": (_i32, [_p, _p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32, _p, _p, _i64,
                                        _i32]),
    "neko_hip_store_kv": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _i32]),
    "neko_hip_attention": (_i32, [_p, _p, _i64, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _i64, _f32, _i32]),
    "neko_hip_add_rmsnorm": (_i32, [_p, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _f32, _i32]),
    "neko_hip_matmul": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i64, _i32, _i64, _p, _p, _i64, _i32, _i32, _i32]),
    "neko_hip_set_matmul_library": (_i32, [_p, _i32]),
    "neko_hip_matmul_noalloc": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i64, _i32, _i64, _p, _p, _i64, _i32, _i32, _i32]),
    "neko_hip_quantize_rows": (_i32, [_p, _i32, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "neko_hip_swiglu": (_i32, [_p, _p, _i64, _p, _i64, _i64, _i64, _i32]),
    "neko_hip_gelu_tanh": (_i32, [_p, _p, _p, _i64, _i32]),
    "neko_hip_embed": (_i32, [_p, _p, _i64, _p, _i64, _i32, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32]),
    "neko_hip_embed_scaled": (_i32, [_p, _p, _i64, _p, _i64, _i32, _i64, _i64, _i64, _f32, _p, _i64, _i32]),
    "neko_quant_row_bytes": (_sz, [_i32, _i64]),
    "neko_quantize_rows": (_i32, [_i32, _i64, _i64, _p, _p, _i32, ctypes.POINTER(_i32)]),
    "neko_rope_table": (_i32, [ctypes.c_double, _i32, _i64, _p]),
}


class NekoError(RuntimeError):
    """A failed neko_hip call (the reference's NekoError, common.h:27-31)."""

    def __init__(self, message: str, code: int = NEKO_ERR_INVALID):
        super().__init__(message)
        self.code = code


def _load() -> ctypes.CDLL:
    # One HIP runtime per process: torch bundles its own libamdhip64 (same SONAME, different file
    # name), so it must be loaded first for libneko_hip.so to bind to it. Loaded the other way round,
    # the process would hold two runtimes and torch's device pointers would be foreign to ours.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the HIP kernels have no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
