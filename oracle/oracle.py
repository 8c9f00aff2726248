"""numpy front end for the CPU oracle (oracle/_build/liboracle.so) and, where it was built, the compiled
reference CPU ops (oracle/_ref/libneko_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the expected results or the timed CPU baseline -- never by the product package.

Arrays: fp16 data travels as numpy uint16 bit patterns (so NaN payloads and -0 survive), f32 as float32.
Every wrapper allocates its outputs and returns them; inputs are never modified unless the name says
"inplace".
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libneko_ref.so")

FMT_F16, FMT_FP8, FMT_FP4 = 0, 1, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float


def build() -> None:
    """Compiles the oracle (and oracle/_ref when the reference checkout is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Lib:
    def __init__(self, path, sigs):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run make -C oracle)")
        self.lib = ctypes.CDLL(path)
        for name, (res, args) in sigs.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    def __getattr__(self, name):
        return getattr(self.lib, name)


_ORACLE_SIGS = {
    "oracle_f16_to_f32": (_f32, [ctypes.c_uint16]),
    "oracle_f32_to_f16": (ctypes.c_uint16, [_f32]),
    "oracle_f16_to_f32_n": (None, [_p, _p, _i64]),
    "oracle_f32_to_f16_n": (None, [_p, _p, _i64]),
    "oracle_gelu": (_f32, [_f32]),
    "oracle_silu": (_f32, [_f32]),
    "oracle_layernorm": (None, [_p, _p, _p, _p, _i32, _i32, _f32]),
    "oracle_rmsnorm": (None, [_p, _p, _p, _i32, _i32, _f32]),
    "oracle_rope": (None, [_p, _i32, _i32, _p]),
    "oracle_silu_mul": (None, [_p, _p, _i32, _i32]),
    "oracle_gated_rmsnorm": (None, [_p, _p, _i64, _p, _i32, _i32, _i32, _f32]),
    "oracle_rope_table": (None, [ctypes.c_double, _i32, _i32, _p]),
    "oracle_quant_row_bytes": (ctypes.c_size_t, [_i32, _i32]),
    "oracle_decode_fp8": (_f32, [ctypes.c_uint8]),
    "oracle_decode_fp4": (_f32, [ctypes.c_uint8]),
    "oracle_encode_fp8": (ctypes.c_uint8, [_f32]),
    "oracle_encode_fp4": (ctypes.c_uint8, [_f32]),
    "oracle_fp4_block_scale": (ctypes.c_uint16, [_p]),
    "oracle_quantize_rows": (_i32, [_i32, _i64, _i32, _p, _p]),
    "oracle_dequantize_row": (None, [_i32, _i32, _p, _p]),
    "oracle_layernorm_f16": (None, [_p, _i64, _p, _i64, _p, _p, _i64, _i32, _f32]),
    "oracle_rmsnorm_f16": (None, [_p, _i64, _p, _i64, _p, _i64, _i32, _f32]),
    "oracle_qk_norm_rope_f16": (None, [_p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32]),
    "oracle_qk_norm_rope_f32": (None, [_p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32]),
    "oracle_swiglu_f16": (None, [_p, _i64, _p, _i64, _i64, _i32]),
    "oracle_gelu_f16": (None, [_p, _p, _i64]),
    "oracle_gated_rmsnorm_f16": (None, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _i32, _f32]),
    "oracle_embed": (None, [_p, _i64, _p, _i64, _i32, _i32, _i64, _i64, _p, _i64, _p, _i64, _i32]),
    "oracle_store_kv": (None, [_p, _p, _i64, _p, _p, _i32, _i64, _i64]),
    "oracle_add_rmsnorm": (None, [_p, _p, _p, _p, _i32, _i32, _f32]),
    "oracle_store_kv_rows": (None, [_p, _i32, _i64, _i64, _i64, _i32, _i64, _i64, _p, _i64, _p, _p]),
    "oracle_qk_norm_rope_kv_f16": (None, [_p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32, _p, _p]),
    "oracle_qk_norm_rope_kv_f32": (None, [_p, _i64, _i64, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _f32, _p, _p]),
    "oracle_add_rmsnorm_f16": (None, [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i32, _f32]),
    "oracle_matmul": (None, [_i32, _p, _i64, _i32, _p, _i64, _i64, _p, _p, _i32]),
    "oracle_attention": (None, [_p, _i64, _p, _p, _p, _i64, _i32, _i32, _i32, _i64]),
}

_REF_SIGS = {
    "ref_f16_to_f32": (_f32, [ctypes.c_uint16]),
    "ref_f32_to_f16": (ctypes.c_uint16, [_f32]),
    "ref_f16_to_f32_n": (None, [_p, _p, _i64]),
    "ref_f32_to_f16_n": (None, [_p, _p, _i64]),
    "ref_gelu": (_f32, [_f32]),
    "ref_layernorm": (None, [_p, _p, _p, _p, _i32, _i32, _f32]),
    "ref_rmsnorm": (None, [_p, _p, _p, _i32, _i32, _f32]),
    "ref_rope": (None, [_p, _i32, _i32, _p]),
    "ref_silu_mul": (None, [_p, _p, _i32, _i32]),
    "ref_quant_row_bytes": (ctypes.c_size_t, [_i32, _i32]),
    "ref_quantize_rows": (_i32, [_i32, _i32, _i32, _p, _p]),
    "ref_dequantize_row": (None, [_i32, _i32, _p, _p]),
    "ref_layernorm_f16": (None, [_p, _p, _p, _p, _i32, _i32, _f32]),
    "ref_rmsnorm_f16": (None, [_p, _p, _p, _i32, _i32, _f32]),
    "ref_qk_norm_rope_f16": (None, [_p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _f32]),
    "ref_silu_mul_f16": (None, [_p, _p, _i32, _i32]),
    "ref_gelu_f16": (None, [_p, _p, _i32]),
    "ref_gated_rmsnorm_f16": (None, [_p, _p, _p, _p, _i32, _i32, _i32, _f32]),
    "ref_embed": (None, [_p, _i32, _p, _i32, _i32, _i32, _p, _i32, _p, _i32]),
    "ref_store_kv": (None, [_p, _p, _i32, _p, _p, _i32, _i32, _i32]),
    "ref_add_rmsnorm_f16": (None, [_p, _p, _p, _p, _p, _i32, _i32, _f32]),
    "ref_gelu_n": (None, [_p, _p, _i64]),
    "ref_matmul": (None, [_i32, _p, _i32, _i32, _p, _i32, _p, _p, _i32]),
    "ref_qk_norm_rope": (None, [_p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _f32]),
    "ref_gated_rmsnorm": (None, [_p, _p, _p, _i32, _i32, _i32, _f32]),
    "ref_qmatrix_new": (_p, [_i32, _i32, _i32, _p]),
    "ref_qmatrix_gather": (None, [_p, _p, _i32, _p, _p]),
    "ref_qmatrix_free": (None, [_p]),
    "ref_qmatrix_matmul": (None, [_p, _p, _i32, _p, _p, _i32]),
    "ref_attention": (None, [_p, _i32, _p, _p, _p, _i32, _i32, _i32, _i32, _i32]),
}

_oracle = None
_ref = None


def lib() -> _Lib:
    global _oracle
    if _oracle is None:
        _oracle = _Lib(ORACLE_SO, _ORACLE_SIGS)
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref() -> _Lib:
    """The compiled reference CPU ops (only where oracle/_ref was built from the reference sources)."""
    global _ref
    if _ref is None:
        _ref = _Lib(REF_SO, _REF_SIGS)
    return _ref


# ------------------------------------------------------------------ conversions

def f16_to_f32(h):
    h = _c16(h)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f):
    f = _c32(f)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_f16_n(_ptr(f), _ptr(out), f.size)
    return out


# ------------------------------------------------------------------ fp16 I/O ops (C-ABI argument meaning)

def layernorm_f16(x, gamma, beta, eps):
    x = _c16(x)
    rows, C = x.shape
    y = np.empty_like(x)
    lib().oracle_layernorm_f16(_ptr(x), C, _ptr(y), C, _ptr(_c32(gamma)), _ptr(_c32(beta)), rows, C, eps)
    return y


def rmsnorm_f16(x, w, eps):
    x = _c16(x)
    rows, C = x.shape
    y = np.empty_like(x)
    lib().oracle_rmsnorm_f16(_ptr(x), C, _ptr(y), C, _ptr(_c32(w)), rows, C, eps)
    return y


def qk_norm_rope_f16(qkv, n_q, n_kv, hd, cs, n_pos, eps, wqk=None, positions=None, pos0=0):
    out = _c16(qkv).copy()
    rows, stride = out.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    w = None if wqk is None else _c32(wqk)
    lib().oracle_qk_norm_rope_f16(_ptr(out), stride, rows, n_q, n_kv, hd, pos0, _ptr(pos), _ptr(w), _ptr(_c32(cs)),
                                  n_pos, eps)
    return out


def qk_norm_rope_f32(qkv, n_q, n_kv, hd, cs, n_pos, eps, wqk=None, positions=None, pos0=0):
    out = _c32(qkv).copy()
    rows, stride = out.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    w = None if wqk is None else _c32(wqk)
    lib().oracle_qk_norm_rope_f32(_ptr(out), stride, rows, n_q, n_kv, hd, pos0, _ptr(pos), _ptr(w), _ptr(_c32(cs)),
                                  n_pos, eps)
    return out


def qk_norm_rope_kv(qkv, n_q, n_kv, hd, cs, n_pos, eps, wqk=None, positions=None, pos0=0):
    """q/k norm + RoPE then the KV store; returns (qkv after, k cache, v cache) with n_pos cache rows
    (rows the op does not write stay 0xFFFF so untouched rows are visible)."""
    f16 = qkv.dtype == np.uint16
    out = (_c16(qkv) if f16 else _c32(qkv)).copy()
    rows, stride = out.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    w = None if wqk is None else _c32(wqk)
    kc = np.full((n_pos, n_kv * hd), 0xFFFF, np.uint16)
    vc = kc.copy()
    fn = lib().oracle_qk_norm_rope_kv_f16 if f16 else lib().oracle_qk_norm_rope_kv_f32
    fn(_ptr(out), stride, rows, n_q, n_kv, hd, pos0, _ptr(pos), _ptr(w), _ptr(_c32(cs)), n_pos, eps, _ptr(kc), _ptr(vc))
    return out, kc, vc


def store_kv(qkv, k_off, v_off, width, cache_rows, positions=None, pos0=0):
    """KV store at the C ABI's meaning; qkv uint16 (f16 bits) or float32. Unwritten cache rows stay 0xFFFF."""
    f16 = qkv.dtype == np.uint16
    src = _c16(qkv) if f16 else _c32(qkv)
    rows, stride = src.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    kc = np.full((cache_rows, width), 0xFFFF, np.uint16)
    vc = kc.copy()
    lib().oracle_store_kv_rows(_ptr(src), int(f16), stride, k_off, v_off, width, rows, pos0, _ptr(pos), cache_rows,
                               _ptr(kc), _ptr(vc))
    return kc, vc


def attention(q, kc, vc, n_head, n_kv, hd, pos0, use_ref=False):
    """cpu::attention's meaning: q float32 [T, q_stride], caches uint16 (f16 bits) [>= pos0 + T, n_kv*hd];
    returns float32 [T, n_head*hd]. use_ref: the compiled reference instead of the restatement."""
    q = _c32(q)
    kc, vc = _c16(kc), _c16(vc)
    T, qs = q.shape
    out = np.empty((T, n_head * hd), np.float32)
    if use_ref:
        ref().ref_attention(_ptr(q), qs, _ptr(kc), _ptr(vc), _ptr(out), T, n_head, n_kv, hd, pos0)
    else:
        lib().oracle_attention(_ptr(q), qs, _ptr(kc), _ptr(vc), _ptr(out), T, n_head, n_kv, hd, pos0)
    return out


def add_rmsnorm_f16(x, d, w, eps):
    """Returns (x + d rounded to f16, rmsnorm of it)."""
    xo = _c16(x).copy()
    d = _c16(d)
    rows, C = xo.shape
    xn = np.empty_like(xo)
    lib().oracle_add_rmsnorm_f16(_ptr(xo), C, _ptr(d), d.shape[1], _ptr(xn), C, _ptr(_c32(w)), rows, C, eps)
    return xo, xn


def swiglu_f16(h):
    h = _c16(h)
    rows, two_i = h.shape
    I = two_i // 2
    out = np.empty((rows, I), np.uint16)
    lib().oracle_swiglu_f16(_ptr(h), two_i, _ptr(out), I, rows, I)
    return out


def gelu_f16(x):
    x = _c16(x)
    y = np.empty_like(x)
    lib().oracle_gelu_f16(_ptr(x), _ptr(y), x.size)
    return y


def gated_rmsnorm_f16(y, z, w, groups, eps):
    y = _c16(y)
    z = _c16(z)
    rows, D = y.shape
    out = np.empty_like(y)
    lib().oracle_gated_rmsnorm_f16(_ptr(y), D, _ptr(z), z.shape[1], _ptr(out), D, _ptr(_c32(w)), rows, D, groups, eps)
    return out


def rope_table(theta, hd, n_pos):
    cs = np.empty((n_pos, hd), np.float32)
    lib().oracle_rope_table(theta, hd, n_pos, _ptr(cs))
    return cs


def quant_row_bytes(fmt, cols):
    return int(lib().oracle_quant_row_bytes(fmt, cols))


def quantize_rows(fmt, x):
    x = _c32(x)
    rows, cols = x.shape
    fmt_used = fmt if cols % 32 == 0 else FMT_F16
    out = np.empty((rows, quant_row_bytes(fmt_used, cols)), np.uint8)
    got = lib().oracle_quantize_rows(fmt, rows, cols, _ptr(x), _ptr(out))
    assert got == fmt_used
    return out


def dequantize_rows(fmt, table, cols):
    table = np.ascontiguousarray(table, dtype=np.uint8)
    out = np.empty((table.shape[0], cols), np.float32)
    for r in range(table.shape[0]):
        lib().oracle_dequantize_row(fmt, cols, _ptr(table[r]), _ptr(out[r]))
    return out


def embed(tokens, table, fmt, C, row_base=0, rows=None, wpe=None, pos0=0, out_f16=True, out=None):
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    table = np.ascontiguousarray(table, dtype=np.uint8)
    rows = table.shape[0] if rows is None else rows
    T = tokens.shape[0]
    if out is None:
        out = np.zeros((T, C), np.uint16 if out_f16 else np.float32)
    pe = None if wpe is None else _c16(wpe)
    lib().oracle_embed(_ptr(tokens), T, _ptr(table), table.shape[1], fmt, C, row_base, rows, _ptr(pe), pos0,
                       _ptr(out), out.shape[1], 1 if out_f16 else 0)
    return out


def matmul(fmt, x, table, K, bias=None, y=None, flags=0):
    """cpu::matmul on the portable path: x float32 [T, K], table uint8 [N, row_bytes] in `fmt`; returns y
    float32 [T, N] (a copy of `y` accumulated into when flags & 2)."""
    x = _c32(x)
    table = np.ascontiguousarray(table, dtype=np.uint8)
    T, N = x.shape[0], table.shape[0]
    out = np.zeros((T, N), np.float32) if y is None else _c32(y).copy()
    b = None if bias is None else _c32(bias)
    lib().oracle_matmul(fmt, _ptr(x), T, K, _ptr(table), table.shape[1], N, _ptr(b), _ptr(out), flags)
    return out
