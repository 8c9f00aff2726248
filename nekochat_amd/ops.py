"""torch-facing host interface to the neko_hip C ABI.

The functions mirror the reference's per-op interface (cpu_ops.h:25-45, quant.h:32-58 and the GPU
dispatches of gpu/compute.h) with torch tensors as the buffers: same op names (snake_case), same
argument meaning, and failures raise NekoError as the reference's fail() does (common.h:27-31).

Activations are 2-D tensors on the GPU with unit stride along the last dimension (any row stride),
dtype float16 or float32. Norm weights are float32 vectors on the same device. Every call runs on
the calling thread's context for the tensor's device, on torch's current stream.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from ._lib import DT_F16, DT_F32, FMT_F16, FMT_FP4, FMT_FP8, NEKO_OK, NekoError, lib

__all__ = [
    "Context", "context", "layer_norm", "rms_norm", "qk_norm_rope", "qk_norm_rope_kv", "store_kv", "add_rms_norm",
    "silu_mul", "gelu", "gated_rms_norm", "embed", "matmul", "MM_GELU", "MM_ACCUMULATE",
    "prepare", "quantize", "quant_row_bytes", "quantize_rows", "rope_table", "FMT_F16", "FMT_FP8", "FMT_FP4", "NekoError",
]


class Context:
    """One neko_hip context: a device and an in-order stream (one per host thread)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        rc = lib.neko_hip_create(int(device), ctypes.byref(h))
        if rc != NEKO_OK:
            raise NekoError(lib.neko_hip_last_error(None).decode(), rc)
        self.handle = h.value
        self.device = int(device)
        self._bound = -1  # stream handle last routed to the C context

    def check(self, rc: int) -> None:
        if rc != NEKO_OK:
            raise NekoError(lib.neko_hip_last_error(self.handle).decode(), rc)

    def bind_torch_stream(self) -> None:
        """Orders the next ops after work already queued on torch's current stream."""
        s = torch.cuda.current_stream(self.device).cuda_stream
        if s != self._bound:  # 0 is the null stream, which the C context uses for NULL too
            self.check(lib.neko_hip_set_stream(self.handle, s or None))
            self._bound = s

    def synchronize(self) -> None:
        self.check(lib.neko_hip_synchronize(self.handle))

    def set_matmul_library(self, enable: bool) -> None:
        """Whether this context's plain F16 prefill matmuls may run on hipBLASLt (default True) or
        stay on the library's own kernels."""
        self.check(lib.neko_hip_set_matmul_library(self.handle, 1 if enable else 0))

    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        self.check(lib.neko_hip_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def close(self) -> None:
        if self.handle:
            lib.neko_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_tls = threading.local()


def context(device: int | None = None) -> Context:
    """The calling thread's context for `device` (default: torch's current device)."""
    if device is None:
        device = torch.cuda.current_device()
    cache = getattr(_tls, "ctx", None)
    if cache is None:
        cache = _tls.ctx = {}
    ctx = cache.get(device)
    if ctx is None:
        ctx = cache[device] = Context(device)
    return ctx


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return DT_F16
    if t.dtype == torch.float32:
        return DT_F32
    raise NekoError(f"activations must be float16 or float32, got {t.dtype}")


def _rows(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise NekoError(f"{name} must be a GPU tensor")
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise NekoError(f"{name} must be 2-D with unit stride along rows, got shape {tuple(t.shape)} "
                        f"strides {t.stride()}")
    return t.shape[0], t.shape[1], t.stride(0)


def _on(t: torch.Tensor | None, name: str, device) -> None:
    """Every buffer handed to the C ABI must live on the op's GPU: a host pointer would reach a kernel."""
    if t is not None and (not t.is_cuda or t.device != device):
        raise NekoError(f"{name} must be a tensor on {device}, got {t.device}")


def _vec(t: torch.Tensor | None, n: int, name: str, device) -> int | None:
    if t is None:
        return None
    if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() < n or t.device != device:
        raise NekoError(f"{name} must be a contiguous float32 GPU vector of at least {n} values on {device}")
    return t.data_ptr()


def _ctx_for(t: torch.Tensor) -> Context:
    ctx = context(t.device.index)
    ctx.bind_torch_stream()
    return ctx


_recording = threading.local()


def _issue(ctx: Context, fn, *args):
    rec = getattr(_recording, "rec", None)
    if rec is not None:  # being prepared: remember the call instead of issuing it
        rec.append((ctx, fn, args))
        return
    ctx.check(fn(*args))


def prepare(op, *args, **kwargs):
    """Validates op(*args, **kwargs) once and returns (run, result): run() re-issues the same C call
    on the same buffers with no Python-side checks -- for tight loops that replay one op. The stream
    is the torch stream current at preparation time."""
    _recording.rec = rec = []
    try:
        result = op(*args, **kwargs)
    finally:
        _recording.rec = None
    if len(rec) != 1:
        raise NekoError(f"prepare: {getattr(op, '__name__', op)} issued {len(rec)} calls; expected one")
    ctx, fn, cargs = rec[0]
    handle, stream = cargs[0], ctx._bound

    def run():
        if ctx._bound != stream:  # another op routed the context elsewhere meanwhile
            ctx.check(lib.neko_hip_set_stream(handle, stream or None))
            ctx._bound = stream
        rc = fn(*cargs)
        if rc != NEKO_OK:
            raise NekoError(lib.neko_hip_last_error(handle).decode(), rc)

    return run, result


def _out_like(x: torch.Tensor, rows: int, cols: int, out: torch.Tensor | None, name: str) -> torch.Tensor:
    if out is None:
        return torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    r, c, _ = _rows(out, name)
    if (r, c) != (rows, cols) or out.dtype != x.dtype or out.device != x.device:
        raise NekoError(f"{name} must be {x.dtype} [{rows}, {cols}] on {x.device}")
    return out


def layer_norm(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """cpu::layerNorm (cpu_ops.cpp:483-500) over the rows of x. out may be x."""
    rows, C, xs = _rows(x, "x")
    out = _out_like(x, rows, C, out, "out")
    ctx = _ctx_for(x)
    _issue(ctx, lib.neko_hip_layernorm, ctx.handle, x.data_ptr(), xs, out.data_ptr(), out.stride(0),
           _vec(gamma, C, "gamma", x.device), _vec(beta, C, "beta", x.device), rows, C,
           float(eps), _dtype_code(x))
    return out


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """cpu::rmsNorm (cpu_ops.cpp:502-511) over the rows of x. out may be x."""
    rows, C, xs = _rows(x, "x")
    out = _out_like(x, rows, C, out, "out")
    ctx = _ctx_for(x)
    _issue(ctx, lib.neko_hip_rmsnorm, ctx.handle, x.data_ptr(), xs, out.data_ptr(), out.stride(0),
           _vec(w, C, "w", x.device), rows, C, float(eps), _dtype_code(x))
    return out


def gated_rms_norm(y: torch.Tensor, z: torch.Tensor, w: torch.Tensor, groups: int, eps: float,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Granite Mamba2 gate + group RMSNorm (granite_model.cpp:278-287): norm(y * silu(z)). z may be
    a column slice of a wider row (only its first D columns are read). out may be y."""
    rows, D, ys = _rows(y, "y")
    zr, zc, zs = _rows(z, "z")
    _on(z, "z", y.device)
    if zr != rows or zc < D or z.dtype != y.dtype:
        raise NekoError(f"z must be {y.dtype} with {rows} rows of at least {D} columns")
    out = _out_like(y, rows, D, out, "out")
    ctx = _ctx_for(y)
    _issue(ctx, lib.neko_hip_gated_rmsnorm, ctx.handle, y.data_ptr(), ys, z.data_ptr(), zs, out.data_ptr(), out.stride(0),
           _vec(w, D, "w", y.device), rows, D, int(groups), float(eps), _dtype_code(y))
    return out


def _rope_inputs(qkv, rows, hd, cs, positions):
    _on(cs, "cs", qkv.device)
    if cs.dtype != torch.float32 or not cs.is_contiguous() or cs.dim() != 2 or cs.shape[1] != hd:
        raise NekoError("cs must be a contiguous float32 [n_pos, hd] table")
    if positions is None:
        return None
    _on(positions, "positions", qkv.device)
    if positions.dtype != torch.int32 or not positions.is_contiguous() or positions.numel() < rows:
        raise NekoError("positions must be a contiguous int32 vector with one entry per row")
    return positions.data_ptr()


def _cache(t: torch.Tensor, rows: int, width: int, name: str, device) -> None:
    _on(t, name, device)
    if t.dtype != torch.float16 or not t.is_contiguous() or t.dim() != 2 or t.shape[1] != width or t.shape[0] < rows:
        raise NekoError(f"{name} must be a contiguous float16 [>= {rows}, {width}] cache")


def qk_norm_rope(qkv: torch.Tensor, n_q: int, n_kv: int, hd: int, cs: torch.Tensor, eps: float,
                 wqk: torch.Tensor | None = None, positions: torch.Tensor | None = None, pos0: int = 0) -> torch.Tensor:
    """Qwen3 q/k head RMSNorm + NeoX RoPE in place on qkv rows (rope.comp; qwen3_model.cpp:249-253).
    cs: float32 [n_pos, hd] cos/sin table (rope_table). positions: int32 [rows] or None for pos0 + row."""
    rows, width, stride = _rows(qkv, "qkv")
    if width < (n_q + n_kv) * hd:
        raise NekoError(f"qkv rows hold {width} values, fewer than {n_q + n_kv} heads x {hd}")
    pos_ptr = _rope_inputs(qkv, rows, hd, cs, positions)
    ctx = _ctx_for(qkv)
    _issue(ctx, lib.neko_hip_qk_norm_rope, ctx.handle, qkv.data_ptr(), stride, rows, int(n_q), int(n_kv), int(hd),
           int(pos0), pos_ptr, _vec(wqk, 2 * hd, "wqk", qkv.device), cs.data_ptr(),
           cs.shape[0], float(eps), _dtype_code(qkv))
    return qkv


def qk_norm_rope_kv(qkv: torch.Tensor, n_q: int, n_kv: int, hd: int, cs: torch.Tensor, eps: float,
                    k_cache: torch.Tensor, v_cache: torch.Tensor, wqk: torch.Tensor | None = None,
                    positions: torch.Tensor | None = None, pos0: int = 0) -> torch.Tensor:
    """qk_norm_rope fused with the KV-cache store that follows it (qwen3_model.cpp:249-256): the
    rotated k heads and the v heads of each row also go to k_cache / v_cache (float16 [>= n_pos,
    n_kv * hd]) at row = the row's position."""
    rows, width, stride = _rows(qkv, "qkv")
    if width < (n_q + 2 * n_kv) * hd:
        raise NekoError(f"qkv rows hold {width} values, fewer than {n_q + 2 * n_kv} heads x {hd}")
    pos_ptr = _rope_inputs(qkv, rows, hd, cs, positions)
    n_pos = cs.shape[0]
    _cache(k_cache, n_pos, n_kv * hd, "k_cache", qkv.device)
    _cache(v_cache, n_pos, n_kv * hd, "v_cache", qkv.device)
    ctx = _ctx_for(qkv)
    _issue(ctx, lib.neko_hip_qk_norm_rope_kv, ctx.handle, qkv.data_ptr(), stride, rows, int(n_q), int(n_kv), int(hd),
           int(pos0), pos_ptr, _vec(wqk, 2 * hd, "wqk", qkv.device), cs.data_ptr(), n_pos, float(eps),
           k_cache.data_ptr(), v_cache.data_ptr(), min(k_cache.shape[0], v_cache.shape[0]), _dtype_code(qkv))
    return qkv


def store_kv(qkv: torch.Tensor, k_off: int, v_off: int, width: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
             positions: torch.Tensor | None = None, pos0: int = 0) -> None:
    """cpu::storeKv (cpu_ops.cpp:535-542): columns [k_off, +width) and [v_off, +width) of each qkv row
    into float16 cache rows positions[t] (or pos0 + t); rows outside the caches are skipped."""
    rows, cols, stride = _rows(qkv, "qkv")
    if k_off < 0 or v_off < 0 or k_off + width > cols or v_off + width > cols:
        raise NekoError("k/v columns exceed the qkv rows")
    cache_rows = min(k_cache.shape[0], v_cache.shape[0])
    _cache(k_cache, 0, width, "k_cache", qkv.device)
    _cache(v_cache, 0, width, "v_cache", qkv.device)
    pos_ptr = None
    if positions is not None:
        _on(positions, "positions", qkv.device)
        if positions.dtype != torch.int32 or not positions.is_contiguous() or positions.numel() < rows:
            raise NekoError("positions must be a contiguous int32 vector with one entry per row")
        pos_ptr = positions.data_ptr()
    ctx = _ctx_for(qkv)
    _issue(ctx, lib.neko_hip_store_kv, ctx.handle, qkv.data_ptr(), stride, int(k_off), int(v_off), rows, int(width),
           int(pos0), pos_ptr, k_cache.data_ptr(), v_cache.data_ptr(), cache_rows, _dtype_code(qkv))


def attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, n_head: int, n_kv: int, hd: int,
              pos0: int = 0, scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """cpu::attention (cpu_ops.cpp:544-575): causal grouped-query attention of the q rows (token t at
    position pos0 + t; head h at columns [h*hd, +hd)) over float16 caches [>= pos0 + T, n_kv*hd]
    holding positions 0 .. pos0 + T - 1. scale defaults to the reference's 1/sqrt(hd). Returns
    [T, n_head*hd] in q's dtype."""
    T, width, qs = _rows(q, "q")
    if n_kv <= 0 or n_head % n_kv:
        raise NekoError("n_head must be a positive multiple of n_kv")
    if width < n_head * hd:
        raise NekoError(f"q rows hold {width} values, fewer than {n_head} heads x {hd}")
    _cache(k_cache, pos0 + T, n_kv * hd, "k_cache", q.device)
    _cache(v_cache, pos0 + T, n_kv * hd, "v_cache", q.device)
    out = _out_like(q, T, n_head * hd, out, "out")
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ctx = _ctx_for(q)
    _issue(ctx, lib.neko_hip_attention, ctx.handle, q.data_ptr(), qs, k_cache.data_ptr(), v_cache.data_ptr(),
           out.data_ptr(), out.stride(0), T, int(n_head), int(n_kv), int(hd), int(pos0), float(scale), _dtype_code(q))
    return out


def add_rms_norm(x: torch.Tensor, delta: torch.Tensor, w: torch.Tensor, eps: float,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Residual add + RMSNorm: x += delta (float add, rounded to x's dtype, in place) -- the
    kAccumulate matmul epilogue, cpu_ops.cpp:123 -- then returns rmsNorm(x) (cpu_ops.cpp:502-511)."""
    rows, C, xs = _rows(x, "x")
    dr, dc, ds = _rows(delta, "delta")
    _on(delta, "delta", x.device)
    if dr != rows or dc != C or delta.dtype != x.dtype:
        raise NekoError(f"delta must be {x.dtype} [{rows}, {C}]")
    out = _out_like(x, rows, C, out, "out")
    ctx = _ctx_for(x)
    _issue(ctx, lib.neko_hip_add_rmsnorm, ctx.handle, x.data_ptr(), xs, delta.data_ptr(), ds, out.data_ptr(),
           out.stride(0), _vec(w, C, "w", x.device), rows, C, float(eps), _dtype_code(x))
    return out


def silu_mul(h: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """cpu::siluMul (cpu_ops.cpp:526-533): rows of h hold gate then up; returns [rows, I]."""
    rows, two_i, hs = _rows(h, "h")
    if two_i % 2:
        raise NekoError("h rows must hold gate and up halves (even width)")
    I = two_i // 2
    out = _out_like(h, rows, I, out, "out")
    ctx = _ctx_for(h)
    _issue(ctx, lib.neko_hip_swiglu, ctx.handle, h.data_ptr(), hs, out.data_ptr(), out.stride(0), rows, I, _dtype_code(h))
    return out


def gelu(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """cpu::gelu (cpu_ops.cpp:20-23) elementwise over a contiguous tensor. out may be x."""
    if not x.is_cuda or not x.is_contiguous():
        raise NekoError("x must be a contiguous GPU tensor")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise NekoError("out must match x")
    ctx = _ctx_for(x)
    _issue(ctx, lib.neko_hip_gelu_tanh, ctx.handle, x.data_ptr(), out.data_ptr(), x.numel(), _dtype_code(x))
    return out


def embed(tokens: torch.Tensor, table: torch.Tensor, fmt: int, C: int, row_base: int = 0, rows: int | None = None,
          wpe: torch.Tensor | None = None, pos0: int = 0, out: torch.Tensor | None = None,
          out_dtype: torch.dtype = torch.float16, scale: float | None = None) -> torch.Tensor:
    """Embedding gather with fused dequantisation (embed.comp, QMatrix::dequantizeRow).
    table: uint8 [rows, row_bytes] in format fmt; tokens: int32 [T]; wpe: float16 [P, C] or None;
    scale: Granite's embedding multiplier, applied in f32 to every dequantised value
    (granite_model.cpp:298-301; not combined with wpe). Tokens outside [row_base, row_base + rows)
    leave their out row untouched."""
    if not tokens.is_cuda:
        raise NekoError("tokens must be a GPU tensor")
    _on(table, "table", tokens.device)
    _on(wpe, "wpe", tokens.device)
    _on(out, "out", tokens.device)
    if tokens.dtype != torch.int32 or not tokens.is_contiguous():
        raise NekoError("tokens must be a contiguous int32 vector")
    if table.dtype != torch.uint8 or table.dim() != 2 or not table.is_contiguous():
        raise NekoError("table must be a contiguous uint8 [rows, row_bytes] tensor")
    T = tokens.numel()
    n_rows = table.shape[0] if rows is None else int(rows)
    if n_rows > table.shape[0]:
        raise NekoError("rows exceeds the table")
    if out is None:
        out = torch.zeros((T, C), dtype=out_dtype, device=tokens.device)
    _, oc, os_ = _rows(out, "out")
    if oc < C:
        raise NekoError("out rows are narrower than C")
    wpe_ptr, wpe_rows = None, 0
    if wpe is not None:
        if wpe.dtype != torch.float16 or not wpe.is_contiguous() or wpe.dim() != 2 or wpe.shape[1] != C:
            raise NekoError("wpe must be a contiguous float16 [P, C] table")
        wpe_ptr, wpe_rows = wpe.data_ptr(), wpe.shape[0]
    ctx = _ctx_for(tokens)
    if scale is not None:
        if wpe is not None:
            raise NekoError("embed: a position table and a multiplier are not combined")
        _issue(ctx, lib.neko_hip_embed_scaled, ctx.handle, tokens.data_ptr(), T, table.data_ptr(), table.shape[1],
               int(fmt), int(C), int(row_base), n_rows, float(scale), out.data_ptr(), os_, _dtype_code(out))
        return out
    _issue(ctx, lib.neko_hip_embed, ctx.handle, tokens.data_ptr(), T, table.data_ptr(), table.shape[1], int(fmt), int(C),
           int(row_base), n_rows, wpe_ptr, wpe_rows, int(pos0), out.data_ptr(), os_,
           _dtype_code(out))
    return out


MM_GELU, MM_ACCUMULATE = 1, 2  # cpu_ops.h MatmulFlags


def matmul(x: torch.Tensor, table: torch.Tensor, fmt: int, K: int, bias: torch.Tensor | None = None,
           out: torch.Tensor | None = None, flags: int = 0, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """cpu::matmul / matmul*.comp (cpu_ops.cpp:474-490): out[t][n] (+)= act(x[t] . W[n] + bias[n]).
    x: float16 or float32 [T, K] rows; table: uint8 [N, row_bytes] weight rows in format fmt; bias: float32
    [N] or None; out: [T, >= N] rows of float32 or float16 (a column slice of a wider buffer is fine).
    flags: MM_GELU applies GELU to the biased sum, MM_ACCUMULATE adds into out."""
    T, xk, xs = _rows(x, "x")
    if xk < K:
        raise NekoError("x rows are narrower than K")
    _on(table, "table", x.device)
    if table.dtype != torch.uint8 or table.dim() != 2 or not table.is_contiguous():
        raise NekoError("table must be a contiguous uint8 [N, row_bytes] tensor")
    N = table.shape[0]
    bias_ptr = _vec(bias, N, "bias", x.device)
    if out is None:
        if flags & MM_ACCUMULATE:
            raise NekoError("MM_ACCUMULATE needs an out tensor to add into")
        out = torch.empty((T, N), dtype=out_dtype, device=x.device)
    _on(out, "out", x.device)
    ot, oc, os_ = _rows(out, "out")
    if ot != T or oc < N:
        raise NekoError(f"out must have {T} rows of at least {N} columns")
    ctx = _ctx_for(x)
    _issue(ctx, lib.neko_hip_matmul, ctx.handle, x.data_ptr(), xs, T, int(K), table.data_ptr(), table.shape[1], int(fmt),
           N, bias_ptr, out.data_ptr(), os_, int(flags), _dtype_code(x), _dtype_code(out))
    return out


def quantize(src: torch.Tensor, fmt: int, out: torch.Tensor | None = None) -> tuple[torch.Tensor, int]:
    """quantizeMatrix (quant.cpp:255-279) on the GPU: float32 or float16 rows [rows, cols] -> uint8 rows of
    quant_row_bytes(fmt_used, cols) in the weight format, bit-identical to the host quantize_rows.
    cols % 32 != 0 stores F16 (fmt_used says so)."""
    rows, cols, stride = _rows(src, "src")
    used = fmt if cols % 32 == 0 else FMT_F16
    rb = quant_row_bytes(used, cols)
    if out is None:
        out = torch.empty((rows, rb), dtype=torch.uint8, device=src.device)
    _on(out, "out", src.device)
    if out.dtype != torch.uint8 or not out.is_contiguous() or tuple(out.shape) != (rows, rb):
        raise NekoError(f"out must be a contiguous uint8 [{rows}, {rb}] tensor")
    got = ctypes.c_int()
    ctx = _ctx_for(src)
    _issue(ctx, lib.neko_hip_quantize_rows, ctx.handle, int(fmt), rows, cols, src.data_ptr(), stride, _dtype_code(src),
           out.data_ptr(), ctypes.byref(got))
    return out, used


# ------------------------------------------------------------------ host-side codecs

def quant_row_bytes(fmt: int, cols: int) -> int:
    """quantRowBytes (quant.cpp:199-208)."""
    return int(lib.neko_quant_row_bytes(int(fmt), int(cols)))


def quantize_rows(fmt: int, x: np.ndarray, threads: int = 0) -> tuple[np.ndarray, int]:
    """quantizeMatrix (quant.cpp:255-279) on host float32 rows; returns (uint8 table, format used)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim != 2:
        raise NekoError("x must be 2-D")
    rows, cols = x.shape
    used = ctypes.c_int()
    fmt_used = fmt if cols % 32 == 0 else FMT_F16
    out = np.empty((rows, quant_row_bytes(fmt_used, cols)), np.uint8)
    rc = lib.neko_quantize_rows(int(fmt), rows, cols, x.ctypes.data_as(ctypes.c_void_p),
                                out.ctypes.data_as(ctypes.c_void_p), int(threads), ctypes.byref(used))
    if rc != NEKO_OK:
        raise NekoError(f"neko_quantize_rows failed ({rc})", rc)
    return out, used.value


def rope_table(theta: float, hd: int, n_pos: int) -> np.ndarray:
    """Qwen3Model::ropeTable (qwen3_model.cpp:102-114): float32 [n_pos, hd] (cos, sin) pairs."""
    cs = np.empty((n_pos, hd), np.float32)
    rc = lib.neko_rope_table(float(theta), int(hd), int(n_pos), cs.ctypes.data_as(ctypes.c_void_p))
    if rc != NEKO_OK:
        raise NekoError(f"neko_rope_table failed ({rc})", rc)
    return cs
