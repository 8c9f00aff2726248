"""Writes tests/golden/golden.npz: small input/output vectors produced by the reference's own compiled CPU
ops (oracle/_ref/libneko_ref.so, built from the reference sources by oracle/Makefile).

Run in the container that holds the reference checkout:  python tests/golden/gen_golden.py
The fixture is data only (numeric arrays, no pickles); tests/test_oracle.py checks the oracle against it
and tests/test_gpu_ops.py checks the HIP kernels against it.

It also writes tests/golden/table_sha256.json: the sha256 of the Qwen3-1.7B-shaped tied table
(151936 x 2048 f32, ~N(0, 0.02), tests/mm_tables.py:qwen3_table_source) and of that table encoded by the
reference's compiled quantizeMatrix into F16, FP8 and FP4 rows, so the full-size encoders can be pinned
without storing 1.1 GB of tables.

Inputs are drawn with numpy's PCG64 (seed 0): normals are rounded to fp16 once; weights are fp16-rounded
then kept as f32, as the reference's loader keeps them.
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle as O  # noqa: E402
from mm_tables import qwen3_table_source  # noqa: E402

P = O._ptr
F = ctypes.c_float


def f16(rng, shape, mean=0.0, std=1.0):
    return (mean + std * rng.standard_normal(shape)).astype(np.float16).view(np.uint16)


def w32(rng, n, mean=1.0, std=0.05):
    return (mean + std * rng.standard_normal(n)).astype(np.float16).astype(np.float32)


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libneko_ref.so is not built (make -C oracle in the container with the reference)")
    R = O.ref()
    rng = np.random.default_rng(0)
    g = {}

    # RMSNorm (cpu_ops.cpp:502-511), Qwen3-0.6B width, plus a zero row and a constant row.
    x = f16(rng, (16, 1024))
    x[3] = 0
    x[4] = np.float16(0.5).view(np.uint16)
    w = w32(rng, 1024)
    y = np.empty_like(x)
    R.ref_rmsnorm_f16(P(x), P(y), P(w), 16, 1024, F(1e-6))
    g.update(rms_x=x, rms_w=w, rms_y=y)

    # LayerNorm (cpu_ops.cpp:483-500), GPT-2 width; rows with a large mean and a constant row.
    x = f16(rng, (8, 768))
    x[2] = (np.float16(100.0) + x[2].view(np.float16)).view(np.uint16)
    x[5] = np.float16(-3.0).view(np.uint16)
    gam, bet = w32(rng, 768, 1.0, 0.02), w32(rng, 768, 0.0, 0.02)
    y = np.empty_like(x)
    R.ref_layernorm_f16(P(x), P(y), P(gam), P(bet), 8, 768, F(1e-5))
    g.update(ln_x=x, ln_g=gam, ln_b=bet, ln_y=y)

    # Qwen3 q/k norm + RoPE (qwen3_model.cpp:249-253): 16 q + 8 kv heads of 128, large positions.
    H, KV, hd, T = 16, 8, 128, 8
    stride = (H + 2 * KV) * hd
    qkv = f16(rng, (T, stride))
    wqk = w32(rng, 2 * hd)
    pos_real = np.array([0, 1, 7, 1000, 2047, 3000, 4095, 4094], np.int32)
    cs = O.rope_table(1e6, hd, 4096)[pos_real].copy()  # table rows for those positions (an input)
    pos = np.arange(T, dtype=np.int32)  # row t uses cs row t
    out = qkv.copy()
    R.ref_qk_norm_rope_f16(P(out), stride, T, H, KV, hd, P(pos), P(wqk[:hd].copy()), P(wqk[hd:].copy()), P(cs), F(1e-6))
    out_nonorm = qkv.copy()
    R.ref_qk_norm_rope_f16(P(out_nonorm), stride, T, H, KV, hd, P(pos), None, None, P(cs), F(1e-6))
    g.update(qk_qkv=qkv, qk_wqk=wqk, qk_cs=cs, qk_pos=pos, qk_out=out, qk_out_nonorm=out_nonorm,
             qk_shape=np.array([H, KV, hd], np.int32))

    # SwiGLU (cpu_ops.cpp:526-533).
    h = f16(rng, (4, 2 * 3072), std=3.0)
    o = np.empty((4, 3072), np.uint16)
    R.ref_silu_mul_f16(P(h), P(o), 4, 3072)
    g.update(swiglu_h=h, swiglu_out=o)

    # GELU tanh (cpu_ops.cpp:20-23) over every fp16 value.
    xs = np.arange(65536, dtype=np.uint16)
    ys = np.empty_like(xs)
    R.ref_gelu_f16(P(xs), P(ys), 65536)
    g.update(gelu_y=ys)

    # Granite gated group RMSNorm (restated gate + compiled rmsNorm), groups 1 and 4.
    yy, zz = f16(rng, (6, 3072)), f16(rng, (6, 3072))
    wg = w32(rng, 3072)
    for groups in (1, 4):
        o = np.empty_like(yy)
        R.ref_gated_rmsnorm_f16(P(yy), P(zz), P(o), P(wg), 6, 3072, groups, F(1e-5))
        g[f"gated_out_g{groups}"] = o
    g.update(gated_y=yy, gated_z=zz, gated_w=wg)

    # Weight codecs: reference quantizeMatrix on f32 weights ~N(0, 0.02) with outliers, then gathers.
    V, C = 64, 256
    wf = (0.02 * rng.standard_normal((V, C))).astype(np.float32)
    wf[5, 17] = 1.5
    wf[9, :32] = 0.0
    wf[11, 40] = -3e-6
    g["quant_src"] = wf
    ids = rng.integers(0, V, 40).astype(np.int32)
    g["embed_ids"] = ids
    for fmt, name in ((0, "f16"), (1, "fp8"), (2, "fp4")):
        rb = int(R.ref_quant_row_bytes(fmt, C))
        tab = np.zeros((V, rb), np.uint8)
        assert R.ref_quantize_rows(fmt, V, C, P(wf), P(tab)) == fmt
        g[f"quant_{name}"] = tab
        o16 = np.zeros((40, C), np.uint16)
        o32 = np.zeros((40, C), np.float32)
        R.ref_embed(P(ids), 40, P(tab), fmt, V, C, None, 0, P(o16), 1)
        R.ref_embed(P(ids), 40, P(tab), fmt, V, C, None, 0, P(o32), 0)
        g[f"embed_{name}_f16"] = o16
        g[f"embed_{name}_f32"] = o32
    # GPT-2 wte + wpe in f32 then one f16 rounding (gpt2_model.cpp:182-187).
    wpe = f16(rng, (48, C), std=0.02)
    o16 = np.zeros((40, C), np.uint16)
    R.ref_embed(P(ids), 40, P(g["quant_f16"]), 0, V, C, P(wpe), 3, P(o16), 1)
    g.update(embed_wpe=wpe, embed_wpe_f16=o16)

    # Decoders over every code (quant.cpp:51-53, 63-65), read back through dequantizeRow.
    row8 = np.zeros(int(R.ref_quant_row_bytes(1, 256)), np.uint8)
    row8[:256] = np.arange(256, dtype=np.uint8)
    row8[256:256 + 16].view(np.uint16)[:] = 0x3C00  # scale 1.0
    dec8 = np.empty(256, np.float32)
    R.ref_dequantize_row(1, 256, P(row8), P(dec8))
    row4 = np.zeros(int(R.ref_quant_row_bytes(2, 32)), np.uint8)
    row4[:16] = (np.arange(16) | (np.arange(16) << 4)).astype(np.uint8)
    row4[16:18].view(np.uint16)[:] = 0x3C00
    dec4 = np.empty(32, np.float32)
    R.ref_dequantize_row(2, 32, P(row4), P(dec4))
    g.update(fp8_decode=dec8, fp4_decode=dec4[:16].copy())

    # KV-cache store (cpu_ops.cpp:535-542): f32 k/v rows of a qkv buffer into f16 caches at pos0 + t,
    # with values that round to f16 subnormals, overflow to inf, and a NaN.
    T, W, stride = 5, 256, 1024
    src = (rng.standard_normal((T, stride)) * 3.0).astype(np.float32)
    src[1, 300] = 1e-6
    src[2, 260] = 70000.0
    src[3, 700] = np.nan
    kc = np.full((12, W), 0xFFFF, np.uint16)
    vc = kc.copy()
    base = src.ctypes.data  # k at column 256, v at column 640 of each 1024-float row
    R.ref_store_kv(ctypes.c_void_p(base + 256 * 4), ctypes.c_void_p(base + 640 * 4), stride, P(kc), P(vc), W, T, 4)
    g.update(kv_src=src, kv_k=kc, kv_v=vc)

    # Residual add + RMSNorm with f16 I/O, through the compiled matmul kAccumulate epilogue and
    # rmsNorm; a row whose sum cancels to zero and a row of large values.
    x, d = f16(rng, (8, 512)), f16(rng, (8, 512), std=0.5)
    d[2] = (-x[2].view(np.float16)).view(np.uint16)
    x[5] = (x[5].view(np.float16) * np.float16(1000.0)).view(np.uint16)
    w = w32(rng, 512)
    xo, xn = np.empty_like(x), np.empty_like(x)
    R.ref_add_rmsnorm_f16(P(x), P(d), P(xo), P(xn), P(w), 8, 512, F(1e-6))
    g.update(addrms_x=x, addrms_d=d, addrms_w=w, addrms_xo=xo, addrms_xn=xn)

    # Weight matmul (cpu::matmul on one thread; x86: matmulF16 / matmulGeneric): f16-valued
    # activations, weights quantised by the compiled quantizeMatrix, bias, each flag combination.
    x = f16(rng, (6, 256)).view(np.float16).astype(np.float32)
    wm = (rng.standard_normal((40, 256)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(40) * 0.1).astype(np.float32)
    y0 = (rng.standard_normal((6, 40))).astype(np.float32)
    g.update(mm_x=x, mm_bias=bias, mm_y0=y0)
    for fmt, name in ((0, "f16"), (1, "fp8"), (2, "fp4")):
        tab = np.zeros((40, int(R.ref_quant_row_bytes(fmt, 256))), np.uint8)
        assert R.ref_quantize_rows(fmt, 40, 256, P(wm), P(tab)) == fmt
        g[f"mm_w_{name}"] = tab
        for flags in (0, 1, 2, 3):
            y = y0.copy()
            R.ref_matmul(fmt, P(x), 6, 256, P(tab), 40, P(bias) if flags != 2 else None, P(y), flags)
            g[f"mm_y_{name}_{flags}"] = y

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **g)
    print(f"wrote {path}: {len(g)} arrays, {os.path.getsize(path)} bytes")
    table_hashes(R)


def table_hashes(R):
    """sha256 of the full-size source table and of its F16 / FP8 / FP4 encodings by quantizeMatrix."""
    x = qwen3_table_source()
    V, C = x.shape
    h = {"rows": V, "cols": C, "source": "tests/mm_tables.py:qwen3_table_source (f32, row-major)",
         "source_sha256": hashlib.sha256(x.data).hexdigest()}
    for fmt, name in ((0, "f16"), (1, "fp8"), (2, "fp4")):
        tab = np.empty((V, int(R.ref_quant_row_bytes(fmt, C))), np.uint8)
        assert R.ref_quantize_rows(fmt, V, C, P(x), P(tab)) == fmt
        h[f"{name}_row_bytes"] = tab.shape[1]
        h[f"{name}_sha256"] = hashlib.sha256(tab.data).hexdigest()
        del tab
    path = os.path.join(HERE, "table_sha256.json")
    with open(path, "w") as f:
        json.dump(h, f, indent=1)
        f.write("\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
