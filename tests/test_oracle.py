"""Pins the CPU oracle (oracle/neko_oracle.c) before anything is checked against it.

1. Golden fixtures written by the reference's own compiled ops (tests/golden/golden.npz): bit-exact.
2. The compiled reference itself (oracle/_ref), where it was built here: bit-exact on fresh seeded inputs.
3. What the mathematics fixes, chosen so that a dropped term, wrong sign/index or transposed operand fails:
   IEEE fp16 conversions exhaustively, closed-form code tables, long-double textbook norms and
   activations, RoPE identities (position 0, norm preservation, the angle table), encoder invariants.
"""
import ctypes
import hashlib
import json
import math
import os

import numpy as np
import pytest

import mm_tables as M
from conftest import f16_line, f32_line
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
P = O._ptr


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


# ------------------------------------------------------------------ 1. golden fixtures

def test_golden_rmsnorm(golden):
    assert np.array_equal(O.rmsnorm_f16(golden["rms_x"], golden["rms_w"], 1e-6), golden["rms_y"])


def test_golden_layernorm(golden):
    assert np.array_equal(O.layernorm_f16(golden["ln_x"], golden["ln_g"], golden["ln_b"], 1e-5), golden["ln_y"])


def test_golden_qk_norm_rope(golden):
    H, KV, hd = (int(v) for v in golden["qk_shape"])
    cs, pos = golden["qk_cs"], golden["qk_pos"]
    got = O.qk_norm_rope_f16(golden["qk_qkv"], H, KV, hd, cs, cs.shape[0], 1e-6, wqk=golden["qk_wqk"], positions=pos)
    assert np.array_equal(got, golden["qk_out"])
    got = O.qk_norm_rope_f16(golden["qk_qkv"], H, KV, hd, cs, cs.shape[0], 1e-6, positions=pos)
    assert np.array_equal(got, golden["qk_out_nonorm"])


def test_golden_swiglu_gelu(golden):
    assert np.array_equal(O.swiglu_f16(golden["swiglu_h"]), golden["swiglu_out"])
    assert np.array_equal(O.gelu_f16(np.arange(65536, dtype=np.uint16)), golden["gelu_y"])


def test_golden_gated(golden):
    for groups in (1, 4):
        got = O.gated_rmsnorm_f16(golden["gated_y"], golden["gated_z"], golden["gated_w"], groups, 1e-5)
        assert np.array_equal(got, golden[f"gated_out_g{groups}"])


@pytest.mark.parametrize("fmt,name", [(0, "f16"), (1, "fp8"), (2, "fp4")])
def test_golden_codecs_and_gather(golden, fmt, name):
    tab = O.quantize_rows(fmt, golden["quant_src"])
    assert np.array_equal(tab, golden[f"quant_{name}"])
    ids = golden["embed_ids"]
    assert np.array_equal(O.embed(ids, tab, fmt, 256), golden[f"embed_{name}_f16"])
    o32 = O.embed(ids, tab, fmt, 256, out_f16=False)
    assert np.array_equal(o32.view(np.uint32), golden[f"embed_{name}_f32"].view(np.uint32))


def test_golden_wpe(golden):
    got = O.embed(golden["embed_ids"], golden["quant_f16"], 0, 256, wpe=golden["embed_wpe"], pos0=3)
    assert np.array_equal(got, golden["embed_wpe_f16"])


def test_golden_store_kv(golden):
    """cpu::storeKv of f32 k/v rows (pos0 4), with values rounding to an f16 subnormal, inf and NaN."""
    kc, vc = O.store_kv(golden["kv_src"], 256, 640, 256, 12, pos0=4)
    assert np.array_equal(kc, golden["kv_k"]) and np.array_equal(vc, golden["kv_v"])


def test_golden_add_rmsnorm(golden):
    """Residual add (compiled matmul kAccumulate epilogue) + compiled rmsNorm, f16 I/O."""
    xo, xn = O.add_rmsnorm_f16(golden["addrms_x"], golden["addrms_d"], golden["addrms_w"], 1e-6)
    assert np.array_equal(xo, golden["addrms_xo"]) and np.array_equal(xn, golden["addrms_xn"])


@pytest.mark.parametrize("fmt,name", [(0, "f16"), (1, "fp8"), (2, "fp4")])
def test_golden_matmul(golden, fmt, name):
    """Compiled cpu::matmul (matmulF16 / matmulGeneric) for each flag combination, bit-exact."""
    for flags in (0, 1, 2, 3):
        bias = golden["mm_bias"] if flags != 2 else None
        y = O.matmul(fmt, golden["mm_x"], golden[f"mm_w_{name}"], 256, bias, golden["mm_y0"], flags)
        assert np.array_equal(y.view(np.uint32), golden[f"mm_y_{name}_{flags}"].view(np.uint32)), flags


def test_golden_decoders(golden):
    d8 = np.array([O.lib().oracle_decode_fp8(c) for c in range(256)], np.float32)
    assert np.array_equal(d8.view(np.uint32), golden["fp8_decode"].view(np.uint32))
    d4 = np.array([O.lib().oracle_decode_fp4(c) for c in range(16)], np.float32)
    assert np.array_equal(d4.view(np.uint32), golden["fp4_decode"].view(np.uint32))


# ------------------------------------------------------------------ 2. the compiled reference

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference checkout here)")


@needs_ref
def test_ref_f16_conversions_exhaustive():
    R = O.ref()
    h = np.arange(65536, dtype=np.uint16)
    a, b = O.f16_to_f32(h), np.empty(65536, np.float32)
    R.ref_f16_to_f32_n(P(h), P(b), 65536)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    rng = np.random.default_rng(1)
    f = (rng.standard_normal(300000) * 10.0 ** rng.integers(-9, 6, 300000)).astype(np.float32)
    f = np.concatenate([f, b[np.isfinite(b)], np.nextafter(b[np.isfinite(b)], np.float32(np.inf))])
    r = np.empty(f.size, np.uint16)
    R.ref_f32_to_f16_n(P(f), P(r), f.size)
    assert np.array_equal(O.f32_to_f16(f), r)


@needs_ref
@pytest.mark.parametrize("seed", [2, 3])
def test_ref_ops_bitexact(seed):
    R = O.ref()
    rng = np.random.default_rng(seed)
    F = ctypes.c_float
    x = (rng.standard_normal((33, 1536)) * 2).astype(np.float16).view(np.uint16)
    w = rng.standard_normal(1536).astype(np.float16).astype(np.float32)
    b = rng.standard_normal(1536).astype(np.float32)
    y = np.empty_like(x)
    R.ref_rmsnorm_f16(P(x), P(y), P(w), 33, 1536, F(1e-5))
    assert np.array_equal(O.rmsnorm_f16(x, w, 1e-5), y)
    R.ref_layernorm_f16(P(x), P(y), P(w), P(b), 33, 1536, F(1e-5))
    assert np.array_equal(O.layernorm_f16(x, w, b, 1e-5), y)
    h = (rng.standard_normal((5, 2000)) * 5).astype(np.float16).view(np.uint16)
    o = np.empty((5, 1000), np.uint16)
    R.ref_silu_mul_f16(P(h), P(o), 5, 1000)
    assert np.array_equal(O.swiglu_f16(h), o)
    H, KV, hd = 4, 2, 64
    qkv = rng.standard_normal((9, (H + 2 * KV) * hd)).astype(np.float16).view(np.uint16)
    cs = O.rope_table(1e4, hd, 100)
    pos = rng.integers(0, 100, 9).astype(np.int32)
    wq = rng.standard_normal(2 * hd).astype(np.float32)
    ref = qkv.copy()
    R.ref_qk_norm_rope_f16(P(ref), qkv.shape[1], 9, H, KV, hd, P(pos), P(wq[:hd].copy()), P(wq[hd:].copy()), P(cs),
                           F(1e-6))
    assert np.array_equal(O.qk_norm_rope_f16(qkv, H, KV, hd, cs, 100, 1e-6, wqk=wq, positions=pos), ref)
    yy = rng.standard_normal((4, 640)).astype(np.float16).view(np.uint16)
    zz = (rng.standard_normal((4, 640)) * 3).astype(np.float16).view(np.uint16)
    wg = rng.standard_normal(640).astype(np.float32)
    for groups in (1, 5):
        o = np.empty_like(yy)
        R.ref_gated_rmsnorm_f16(P(yy), P(zz), P(o), P(wg), 4, 640, groups, F(1e-5))
        assert np.array_equal(O.gated_rmsnorm_f16(yy, zz, wg, groups, 1e-5), o)
    xs = rng.standard_normal(4096).astype(np.float32) * 6
    assert np.array_equal(np.array([O.lib().oracle_gelu(v) for v in xs], np.float32).view(np.uint32),
                          np.array([R.ref_gelu(v) for v in xs], np.float32).view(np.uint32))
    # KV store: f32 rows of a qkv buffer (k at 100, v at 900, width 300) into caches at pos0 + t.
    src = (rng.standard_normal((7, 1300)) * 4).astype(np.float32)
    src[2, 150] = 3e5
    kc = np.full((20, 300), 0xFFFF, np.uint16)
    vc = kc.copy()
    R.ref_store_kv(ctypes.c_void_p(src.ctypes.data + 400), ctypes.c_void_p(src.ctypes.data + 3600), 1300, P(kc), P(vc),
                   300, 7, 11)
    ok, ov = O.store_kv(src, 100, 900, 300, 20, pos0=11)
    assert np.array_equal(ok, kc) and np.array_equal(ov, vc)
    # Residual add + RMSNorm (compiled kAccumulate epilogue and rmsNorm).
    x = (rng.standard_normal((6, 384)) * 3).astype(np.float16).view(np.uint16)
    d = rng.standard_normal((6, 384)).astype(np.float16).view(np.uint16)
    w3 = rng.standard_normal(384).astype(np.float16).astype(np.float32)
    xo, xn = np.empty_like(x), np.empty_like(x)
    R.ref_add_rmsnorm_f16(P(x), P(d), P(xo), P(xn), P(w3), 6, 384, F(1e-5))
    oxo, oxn = O.add_rmsnorm_f16(x, d, w3, 1e-5)
    assert np.array_equal(oxo, xo) and np.array_equal(oxn, xn)


@needs_ref
def test_ref_f32_entry_points_match_oracle():
    """The f32-activation forms the CPU baseline times compute what the oracle's f32 functions do."""
    R = O.ref()
    L = O.lib()
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(5000) * 6).astype(np.float32)
    a, b = np.empty_like(x), np.empty_like(x)
    R.ref_gelu_n(P(x), P(a), x.size)
    b[:] = [L.oracle_gelu(v) for v in x]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    H, KV, hd, T = 4, 2, 64, 9
    stride = (H + 2 * KV) * hd
    qkv = rng.standard_normal((T, stride)).astype(np.float32)
    cs = O.rope_table(1e4, hd, 100)
    pos = rng.integers(0, 100, T).astype(np.int32)
    wqk = rng.standard_normal(2 * hd).astype(np.float32)
    r, o = qkv.copy(), qkv.copy()
    R.ref_qk_norm_rope(P(r), stride, T, H, KV, hd, P(pos), P(wqk[:hd].copy()), P(wqk[hd:].copy()), P(cs),
                       ctypes.c_float(1e-6))
    L.oracle_qk_norm_rope_f32(P(o), stride, T, H, KV, hd, 0, P(pos), P(wqk), P(cs), 100, 1e-6)
    assert np.array_equal(r.view(np.uint32), o.view(np.uint32))
    assert not np.array_equal(r, qkv)
    y = rng.standard_normal((4, 640)).astype(np.float32)
    z = (rng.standard_normal((4, 640)) * 3).astype(np.float32)
    wg = rng.standard_normal(640).astype(np.float32)
    for groups in (1, 5):
        r, o = y.copy(), y.copy()
        R.ref_gated_rmsnorm(P(r), P(z), P(wg), 4, 640, groups, ctypes.c_float(1e-5))
        L.oracle_gated_rmsnorm(P(o), P(z), 640, P(wg), 4, 640, groups, 1e-5)
        assert np.array_equal(r.view(np.uint32), o.view(np.uint32))
    cols, rows = 256, 50
    src = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    ids = rng.integers(0, rows, 17).astype(np.int32)
    wpe = rng.standard_normal((17, cols)).astype(np.float32)
    for fmt in (0, 1, 2):
        tab = O.quantize_rows(fmt, src)
        h = R.ref_qmatrix_new(fmt, rows, cols, P(tab))
        try:
            for pe in (None, wpe):
                got = np.empty((17, cols), np.float32)
                R.ref_qmatrix_gather(h, P(ids), 17, P(pe), P(got))
                want = np.empty_like(got)
                for t, i in enumerate(ids):
                    L.oracle_dequantize_row(fmt, cols, P(tab[i]), P(want[t]))
                if pe is not None:
                    want += pe
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        finally:
            R.ref_qmatrix_free(h)


@needs_ref
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_ref_matmul_bitexact(fmt):
    R = O.ref()
    rng = np.random.default_rng(40 + fmt)
    for T, K, N in ((1, 64, 7), (5, 256, 33), (9, 96, 4), (4, 32, 1)):
        if fmt != 0 and K % 32:
            continue
        w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
        tab = O.quantize_rows(fmt, w)
        x = rng.standard_normal((T, K)).astype(np.float16).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        for flags in (0, 1, 2, 3):
            for bias in (None, b):
                y0 = rng.standard_normal((T, N)).astype(np.float32)
                want = y0.copy()
                R.ref_matmul(fmt, P(x), T, K, P(tab), N, P(bias), P(want), flags)
                got = O.matmul(fmt, x, tab, K, bias, y0, flags)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (T, K, N, flags, bias is None)


@needs_ref
@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("cols,scale", [(256, 0.02), (1024, 1.0), (96, 1e-4), (100, 0.02), (64, 3e4)])
def test_ref_quantizer_bitexact(fmt, cols, scale):
    R = O.ref()
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((40, cols)) * scale).astype(np.float32)
    x[0, :] = 0
    x[1, 3] = scale * 50
    x[2, :] = rng.standard_t(2, cols) * scale
    got = O.quantize_rows(fmt, x)
    want = np.zeros_like(got)
    R.ref_quantize_rows(fmt, 40, cols, P(x), P(want))
    assert np.array_equal(got, want)
    used = fmt if cols % 32 == 0 else 0
    for r in range(0, 40, 7):
        a, b = np.empty(cols, np.float32), np.empty(cols, np.float32)
        O.lib().oracle_dequantize_row(used, cols, P(got[r]), P(a))
        R.ref_dequantize_row(used, cols, P(got[r]), P(b))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_full_table_encodings_match_reference_sha256():
    """The oracle's encoder over the full Qwen3-1.7B tied table (151936 x 2048 f32) gives the same bytes
    as the reference's compiled quantizeMatrix, pinned by the sha256 values it wrote
    (tests/golden/table_sha256.json) -- every row, block scale, code and padding byte at full size."""
    with open(os.path.join(os.path.dirname(GOLDEN), "table_sha256.json")) as f:
        want = json.load(f)
    x = M.qwen3_table_source(want["rows"], want["cols"])
    assert hashlib.sha256(x.data).hexdigest() == want["source_sha256"], "source table generator changed"
    for fmt, name in ((0, "f16"), (1, "fp8"), (2, "fp4")):
        tab = O.quantize_rows(fmt, x)
        assert tab.shape[1] == want[f"{name}_row_bytes"]
        assert hashlib.sha256(tab.data).hexdigest() == want[f"{name}_sha256"], name
        del tab


# ------------------------------------------------------------------ 3. what the mathematics fixes

def test_f16_widen_is_ieee():
    h = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(O.f16_to_f32(h).view(np.uint32), h.view(np.float16).astype(np.float32).view(np.uint32))


def test_f16_narrow_is_ieee_rne():
    rng = np.random.default_rng(4)
    f = (rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000)).astype(np.float32)
    edges = np.array([65504, 65519.996, 65520, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0000001, 2 ** -14, np.inf, -0.0],
                     np.float32)
    f = np.concatenate([f, edges, -edges])
    assert np.array_equal(O.f32_to_f16(f), f.astype(np.float16).view(np.uint16))
    nan = np.array([np.nan, -np.nan], np.float32)
    assert list(O.f32_to_f16(nan)) == [0x7E00, 0xFE00]


def _e4m3(c):
    s = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 0xF, c & 7
    return s * (2.0 ** -6 * m / 8 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8))


def test_fp8_code_table_closed_form():
    got = np.array([O.lib().oracle_decode_fp8(c) for c in range(256)])
    want = np.array([_e4m3(c) for c in range(256)])
    assert np.array_equal(got, want)  # includes 0x7F -> 480, 0xFF -> -480 (no NaN code)
    assert math.copysign(1, got[0x80]) == -1 and got[0x80] == 0


def test_fp4_code_table_closed_form():
    mags = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    got = [O.lib().oracle_decode_fp4(c) for c in range(16)]
    assert got == mags + [-m for m in mags]
    assert math.copysign(1, got[8]) == -1


def test_quant_row_bytes_closed_form():
    for cols in (32, 64, 96, 256, 768, 2048, 4096):
        nb = cols // 32
        pad = -(-2 * nb // 16) * 16
        assert O.quant_row_bytes(0, cols) == 2 * cols
        assert O.quant_row_bytes(1, cols) == cols + pad
        assert O.quant_row_bytes(2, cols) == cols // 2 + pad
    assert O.quant_row_bytes(1, 2048) == 2176 and O.quant_row_bytes(2, 2048) == 1152


def test_fp8_encoder_invariants():
    """Scale = RNE_f16(amax / 448). Each code is x * (1/scale) rounded to fp16 first and then to the
    nearest E4M3 value, ties to the even code (the reference rounds twice, quant.cpp:43-49); the sign bit
    is the sign of x."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((50, 64)) * 0.05).astype(np.float32)
    x[0, :8] = [-0.0, 0.0, -1e-30, 1e-30, 0.05, -0.05, 0.025, -0.0125]
    tab = O.quantize_rows(1, x)
    grid = np.array([_e4m3(c) for c in range(0x7F)])
    for r in range(50):
        for b in range(2):
            blk = x[r, 32 * b:32 * b + 32]
            s_bits = int(tab[r, 64 + 2 * b]) | (int(tab[r, 65 + 2 * b]) << 8)
            assert s_bits == int(np.float16(np.abs(blk).max() / np.float32(448)).view(np.uint16))
            inv = np.float32(1) / np.float32(np.uint16(s_bits).view(np.float16))
            for i, v in enumerate(blk):
                c = int(tab[r, 32 * b + i])
                q16 = abs(float(np.float16(np.float32(v) * inv * np.float32(1 / 256)))) * 256
                d = np.abs(grid - q16)
                best = np.flatnonzero(d == d.min())
                assert (c & 0x7F) in best
                if len(best) == 2:
                    assert (c & 1) == 0  # tie -> even mantissa
                assert bool(c & 0x80) == bool(np.signbit(v))


def test_fp4_scale_is_best_of_candidates():
    """The FP4 block scale is amax/6 or a least-squares refit, never worse (squared error) than amax/6."""
    rng = np.random.default_rng(6)
    mags = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    for _ in range(200):
        blk = (rng.standard_normal(32) * 0.02).astype(np.float32)
        s = float(np.uint16(O.lib().oracle_fp4_block_scale(P(blk))).view(np.float16))
        s0 = float(np.float16(np.abs(blk).max() / np.float32(6)))

        def err(sc):
            q = np.abs(blk) / sc
            r = mags[np.abs(q[:, None] - mags[None, :]).argmin(1)]
            return float(((np.abs(blk) - r * sc) ** 2).sum())

        assert err(s) <= err(s0) * (1 + 1e-5) + 1e-18


def _ld(a):
    return np.asarray(a, dtype=np.longdouble)


def test_rmsnorm_textbook():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((20, 2560)) * 3).astype(np.float32)
    x[4] = 0
    w = (1 + 0.05 * rng.standard_normal(2560)).astype(np.float32)
    y = np.empty_like(x)
    O.lib().oracle_rmsnorm(P(x), P(y), P(w), 20, 2560, 1e-6)
    xl = _ld(x)
    want = xl / np.sqrt((xl * xl).mean(1, keepdims=True) + _ld(np.float32(1e-6))) * _ld(w)
    np.testing.assert_allclose(y.astype(np.float64), want.astype(np.float64), rtol=4e-7, atol=0)
    assert not y[4].any()


def test_layernorm_textbook():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((20, 768)) + 50).astype(np.float32)
    x[3] = 7.25  # constant row: output = beta
    g = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    b = (0.02 * rng.standard_normal(768)).astype(np.float32)
    y = np.empty_like(x)
    O.lib().oracle_layernorm(P(x), P(y), P(g), P(b), 20, 768, 1e-5)
    xl = _ld(x)
    mu = xl.mean(1, keepdims=True)
    want = (xl - mu) / np.sqrt(((xl - mu) ** 2).mean(1, keepdims=True) + _ld(np.float32(1e-5))) * _ld(g) + _ld(b)
    np.testing.assert_allclose(y.astype(np.float64), want.astype(np.float64), rtol=0, atol=3e-6)
    assert np.array_equal(y[3], b)


def test_gelu_silu_textbook():
    xs = np.linspace(-12, 12, 4001).astype(np.float32)
    got = np.array([O.lib().oracle_gelu(v) for v in xs])
    xl = _ld(xs)
    inner = _ld(np.float32(0.7978845608)) * (xl + _ld(np.float32(0.044715)) * xl ** 3)
    want = 0.5 * xl * (1 + np.tanh(inner))
    # 1 + tanh cancels for x << 0: the bound adds a few f32 ulps of 1 scaled by |x|.
    assert np.all(np.abs(got - want.astype(np.float64)) <= 2e-6 * np.abs(want.astype(np.float64)) + np.abs(xs) * 2.0 ** -23)
    assert O.lib().oracle_gelu(0.0) == 0.0
    sil = np.array([O.lib().oracle_silu(v) for v in xs])
    np.testing.assert_allclose(sil, (xl / (1 + np.exp(-xl))).astype(np.float64), rtol=1e-6, atol=1e-30)
    assert np.all(got[xs > 6] == xs[xs > 6])  # tanh saturates to 1 in float: gelu(x) = x


def _gated_textbook(y, z, w, groups, eps, mistake=None):
    """granite_model.cpp:21,278-287 from the formulas, in long double: g = y * z / (1 + e^-z), then for
    each of `groups` slices of D / groups channels, g * w[slice] / sqrt(mean(g^2) + eps).
    `mistake` builds a plausible wrong composition instead: "silu_y" (silu applied to y, not z),
    "unsliced" (every group takes the first slice of w), "norm_before_gate" (norm y, then gate),
    "gate_f16" (the gate rounded to fp16 before the norm)."""
    yl, zl = _ld(y), _ld(z)
    if mistake == "silu_y":
        g = yl / (1 + np.exp(-yl)) * zl
    elif mistake == "norm_before_gate":
        g = yl
    else:
        g = yl * (zl / (1 + np.exp(-zl)))
    if mistake == "gate_f16":
        g = _ld(g.astype(np.float64).astype(np.float16))
    D = g.shape[1]
    GS = D // groups
    out = np.empty_like(g)
    for k in range(groups):
        s = slice(k * GS, (k + 1) * GS)
        wk = _ld(w[:GS] if mistake == "unsliced" else w[s])
        gk = g[:, s]
        out[:, s] = gk / np.sqrt((gk * gk).mean(1, keepdims=True) + _ld(np.float32(eps))) * wk
    if mistake == "norm_before_gate":
        out = out * (zl / (1 + np.exp(-zl)))
    return out


@pytest.mark.parametrize("groups", [1, 3, 4])
def test_gated_rmsnorm_textbook(groups):
    """Pins the gate composition of the Granite gated norm independently of any restatement of it:
    which operand takes silu, the f32 gate kept unrounded before the norm, and each group normed
    with its own slice of the weights. Every listed mistake falls outside the tolerance."""
    rng = np.random.default_rng(20 + groups)
    rows, D, eps = 12, 768, 1e-5
    GS = D // groups
    y = (rng.standard_normal((rows, D)) * 2).astype(np.float16).astype(np.float32)
    zfull = (rng.standard_normal((rows, D + 64)) * 3 - 0.5).astype(np.float16).astype(np.float32)
    z = zfull[:, 16:16 + D]  # a column slice of a wider row, as the gate columns of in_proj are
    # Distinct weights per group, so a wrong slice changes every group after the first.
    w = np.concatenate([(1 + 0.4 * k + 0.05 * rng.standard_normal(GS)) for k in range(groups)]).astype(np.float32)

    # f32 activations: the reference's own type. Error budget: expf, the quotient, the product, the
    # float scale and two float multiplies, each within an ulp or so.
    got = y.copy()
    zp = ctypes.c_void_p(zfull.ctypes.data + 16 * 4)
    O.lib().oracle_gated_rmsnorm(P(got), zp, D + 64, P(w), rows, D, groups, eps)

    def within(out):
        ref = out.astype(np.float64)
        return np.all(np.abs(got.astype(np.float64) - ref) <= 2e-6 * np.abs(ref) + 1e-7)

    assert within(_gated_textbook(y, z, w, groups, eps))
    wrong = ["silu_y", "norm_before_gate", "gate_f16"] + (["unsliced"] if groups > 1 else [])
    for m in wrong:
        assert not within(_gated_textbook(y, z, w, groups, eps, mistake=m)), m

    # fp16 I/O: within 1 fp16 ulp of the long-double value rounded to fp16; the coarse mistakes are
    # far outside 2 ulp.
    y16 = y.astype(np.float16).view(np.uint16)
    z16 = np.ascontiguousarray(z).astype(np.float16).view(np.uint16)
    got16 = O.gated_rmsnorm_f16(y16, z16, w, groups, eps)

    def ulps(out):
        want = out.astype(np.float64).astype(np.float16).view(np.uint16)
        return np.abs(f16_line(got16) - f16_line(want))

    assert ulps(_gated_textbook(y, z, w, groups, eps)).max() <= 1
    for m in ["silu_y", "norm_before_gate"] + (["unsliced"] if groups > 1 else []):
        assert ulps(_gated_textbook(y, z, w, groups, eps, mistake=m)).max() > 2, m


def test_rope_identities():
    hd, n_pos = 128, 4096
    cs = O.rope_table(1e6, hd, n_pos)
    c, s = cs[:, 0::2].astype(np.float64), cs[:, 1::2].astype(np.float64)
    assert np.all(np.abs(c * c + s * s - 1) < 2.5e-7)
    assert np.array_equal(cs[0, 0::2], np.ones(64, np.float32)) and not cs[0, 1::2].any()
    p = np.arange(n_pos, dtype=np.float64)
    assert np.all(np.abs(f32_line(cs[:, 0]) - f32_line(np.cos(p).astype(np.float32))) <= 1)  # i = 0: angle p
    assert np.all(np.abs(f32_line(cs[:, 1]) - f32_line(np.sin(p).astype(np.float32))) <= 1)
    inv = 1e6 ** (-2.0 * 63 / hd)
    ang = p * inv
    assert np.all(np.abs(f32_line(cs[:, 126]) - f32_line(np.cos(ang).astype(np.float32))) <= 1)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, hd)).astype(np.float32)
    v = x.copy()
    O.lib().oracle_rope(P(v), 3, hd, P(cs[0]))
    assert np.array_equal(v, x)  # position 0 rotates nothing
    v = x.copy()
    O.lib().oracle_rope(P(v), 3, hd, P(cs[1234]))
    before = x[:, :64] ** 2 + x[:, 64:] ** 2
    after = v[:, :64].astype(np.float64) ** 2 + v[:, 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(after, before, rtol=2e-6)
    # pair i of the first half rotates with pair i of the second half (NeoX split), by angle pos * inv_i
    a, b = x[0, 5], x[0, 69]
    cc, ss = cs[1234, 10], cs[1234, 11]
    assert v[0, 5] == np.float32(a * cc) - np.float32(b * ss)
    assert v[0, 69] == np.float32(a * ss) + np.float32(b * cc)


def test_store_kv_closed_form():
    """The KV store is numpy's IEEE RNE cast to f16 of each k/v value, written at the row's position;
    f16 activations are copied bit for bit; rows outside the cache are skipped."""
    rng = np.random.default_rng(21)
    src = (rng.standard_normal((9, 700)) * 300).astype(np.float32)
    src[0, 50:54] = [np.inf, -np.inf, 1e-8, -7e4]
    pos = np.array([3, 0, 8, -1, 5, 12, 7, 1, 2], np.int32)  # -1 and 12 are outside 10 cache rows
    kc, vc = O.store_kv(src, 40, 400, 256, 10, positions=pos)
    for t, p in enumerate(pos):
        if 0 <= p < 10:
            assert np.array_equal(kc[p], src[t, 40:296].astype(np.float16).view(np.uint16))
            assert np.array_equal(vc[p], src[t, 400:656].astype(np.float16).view(np.uint16))
    assert (kc[[4, 6, 9]] == 0xFFFF).all()  # rows no token maps to stay untouched
    h = rng.integers(0, 65536, (4, 64), dtype=np.uint16)
    kh, vh = O.store_kv(h, 0, 32, 32, 6, pos0=2)
    assert np.array_equal(kh[2:6], h[:, :32]) and np.array_equal(vh[2:6], h[:, 32:])


def test_add_rmsnorm_closed_form():
    """The residual sum is numpy's f32 add of the widened halves rounded to f16; the norm is the
    oracle's (pinned) rmsnorm of that stored sum, and a cancelling row gives the eps-only scale."""
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((5, 300)) * 8).astype(np.float16)
    d = (rng.standard_normal((5, 300)) * 0.01).astype(np.float16)
    d[3] = -x[3]
    w = rng.standard_normal(300).astype(np.float16).astype(np.float32)
    xo, xn = O.add_rmsnorm_f16(x.view(np.uint16), d.view(np.uint16), w, 1e-6)
    want = (x.astype(np.float32) + d.astype(np.float32)).astype(np.float16).view(np.uint16)
    assert np.array_equal(xo, want)
    assert np.array_equal(xn, O.rmsnorm_f16(want, w, 1e-6))
    assert (xo[3] == 0).all() and (xn[3].view(np.float16) == 0).all()  # +0 sums; -0 where w < 0


def test_qk_norm_rope_kv_is_rope_then_store():
    """The fused form equals q/k norm + RoPE followed by the KV store of the rotated rows."""
    rng = np.random.default_rng(23)
    H, KV, hd, n_pos = 4, 2, 64, 40
    qkv = rng.standard_normal((11, (H + 2 * KV) * hd)).astype(np.float16).view(np.uint16)
    cs = O.rope_table(1e6, hd, n_pos)
    wq = rng.standard_normal(2 * hd).astype(np.float32)
    pos = rng.permutation(n_pos)[:11].astype(np.int32)
    pos[4] = n_pos  # out of range: untouched, stores nothing
    out, kc, vc = O.qk_norm_rope_kv(qkv, H, KV, hd, cs, n_pos, 1e-6, wqk=wq, positions=pos)
    rot = O.qk_norm_rope_f16(qkv, H, KV, hd, cs, n_pos, 1e-6, wqk=wq, positions=pos)
    assert np.array_equal(out, rot)
    kw = KV * hd
    for t, p in enumerate(pos):
        if p < n_pos:
            assert np.array_equal(kc[p], rot[t, H * hd:H * hd + kw])
            assert np.array_equal(vc[p], qkv[t, H * hd + kw:H * hd + 2 * kw])
    assert np.count_nonzero((kc != 0xFFFF).any(axis=1)) == 10
    f32 = rng.standard_normal((3, (H + 2 * KV) * hd)).astype(np.float32)
    o32, k32, v32 = O.qk_norm_rope_kv(f32, H, KV, hd, cs, n_pos, 1e-6, wqk=wq, pos0=5)
    r32 = O.qk_norm_rope_f32(f32, H, KV, hd, cs, n_pos, 1e-6, wqk=wq, pos0=5)
    assert np.array_equal(o32, r32)
    assert np.array_equal(k32[5:8], r32[:, H * hd:H * hd + kw].astype(np.float16).view(np.uint16))
    assert np.array_equal(v32[5:8], f32[:, H * hd + kw:].astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------ weight matmul

@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_matmul_integer_rows_exact(fmt):
    """Integer weights (codes times power-of-two scales) and integer activations: every partial sum
    is exact, so the matmul equals the integer dot product; GELU and accumulate apply to that value."""
    import mm_tables as M

    rng = np.random.default_rng(60 + fmt)
    T, K, N = 7, 320, 19
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    exact = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float64) + bias
    assert np.array_equal(O.matmul(fmt, x, tab, K, bias), exact.astype(np.float32))
    g = O.matmul(fmt, x, tab, K, bias, None, 1)
    want = np.array([O.lib().oracle_gelu(float(v)) for v in exact.ravel()], np.float32).reshape(T, N)
    assert np.array_equal(g.view(np.uint32), want.view(np.uint32))
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    a = O.matmul(fmt, x, tab, K, None, y0, 2)
    assert np.array_equal(a, y0 + (exact - bias).astype(np.float32))


@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_matmul_float_within_summation_bound(fmt):
    """Random rows: within K * 2^-24 * sum|x_k w_k| of the float64 product of the dequantised weights
    (the bound of a sequential f32 sum), and far from it when one term is dropped."""
    import mm_tables as M

    rng = np.random.default_rng(70 + fmt)
    T, K, N = 3, 512, 24
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    tab = O.quantize_rows(fmt, w)
    wd = M.dequant(fmt, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float16).astype(np.float32)
    exact, mag = M.exact_and_bound(x, wd)
    err = np.abs(O.matmul(fmt, x, tab, K).astype(np.float64) - exact)
    assert (err <= (K + 1) * 2.0 ** -24 * mag).all()
    x2 = x.copy()
    x2[:, 100] = 0.0
    dropped = np.abs(O.matmul(fmt, x2, tab, K).astype(np.float64) - exact)
    assert (dropped > (K + 1) * 2.0 ** -24 * mag)[np.abs(x[:, 100:101] * wd[None, :, 100]) > 1e-3 * mag].all()



ATTN_SHAPES = [(3, 4, 2, 64, 1030), (1, 32, 8, 128, 300), (5, 12, 12, 64, 7), (2, 6, 2, 96, 40), (4, 3, 1, 256, 20),
               (3, 4, 2, 6, 9)]


def _attn_inputs(T, H, KV, hd, pos0, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, (H + 2 * KV) * hd)).astype(np.float32)
    kc = rng.standard_normal((pos0 + T, KV * hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((pos0 + T, KV * hd)).astype(np.float16).view(np.uint16)
    return q, kc, vc


@needs_ref
@pytest.mark.parametrize("T,H,KV,hd,pos0", ATTN_SHAPES)
def test_ref_attention_bitexact(T, H, KV, hd, pos0):
    """The restatement is the compiled cpu::attention bit for bit (the same summation orders)."""
    q, kc, vc = _attn_inputs(T, H, KV, hd, pos0, T * 7 + hd)
    got = O.attention(q, kc, vc, H, KV, hd, pos0)
    want = O.attention(q, kc, vc, H, KV, hd, pos0, use_ref=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _attn_f64(q, kc, vc, H, KV, hd, pos0, kv_of=None, scale=None, extra=0):
    """Textbook causal softmax attention in float64: head h reads kv head kv_of(h) of rows 0 .. pos0 + t
    (+ extra), scores scaled by 1/sqrt(hd)."""
    kv_of = kv_of or (lambda h: h // (H // KV))
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    k = kc.view(np.float16).astype(np.float64)
    v = vc.view(np.float16).astype(np.float64)
    T = q.shape[0]
    out = np.empty((T, H * hd))
    for t in range(T):
        L = min(pos0 + t + 1 + extra, k.shape[0])
        for h in range(H):
            g = kv_of(h)
            s = k[:L, g * hd:(g + 1) * hd] @ q[t, h * hd:(h + 1) * hd].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ v[:L, g * hd:(g + 1) * hd]
    return out


@pytest.mark.parametrize("T,H,KV,hd,pos0", ATTN_SHAPES)
def test_attention_float64_softmax(T, H, KV, hd, pos0):
    """Within 1e-5 of a float64 softmax attention with the grouped-query head mapping h -> h / (H / KV);
    a wrong mapping (h % KV), a missing scale or one key too many each miss it by far."""
    q, kc, vc = _attn_inputs(T, H, KV, hd, pos0, T * 5 + hd)
    got = O.attention(q, kc, vc, H, KV, hd, pos0).astype(np.float64)
    rel = lambda a: np.abs(got - a) / (1.0 + np.abs(a))  # noqa: E731
    assert rel(_attn_f64(q, kc, vc, H, KV, hd, pos0)).max() <= 1e-5
    if KV > 1 and H // KV > 1:
        assert rel(_attn_f64(q, kc, vc, H, KV, hd, pos0, kv_of=lambda h: h % KV)).max() > 1e-2
    assert rel(_attn_f64(q, kc, vc, H, KV, hd, pos0, scale=1.0)).max() > 1e-2
    if T > 1:  # one more key than the causal range (the last token has no later row)
        assert rel(_attn_f64(q, kc, vc, H, KV, hd, pos0, extra=1)).max() > 1e-3


def test_attention_closed_forms():
    """Position 0 sees one key: out = v_0 bit for bit. Equal keys weight every row alike: out = the
    f32 mean of the v rows, within a few ulp."""
    q, kc, vc = _attn_inputs(1, 4, 2, 64, 0, 31)
    out = O.attention(q, kc, vc, 4, 2, 64, 0)
    v0 = vc[0].view(np.float16).astype(np.float32)
    assert np.array_equal(out[0], np.concatenate([v0[:64], v0[:64], v0[64:], v0[64:]]))
    T, pos0 = 2, 50
    q, kc, vc = _attn_inputs(T, 4, 2, 64, pos0, 32)
    kc[:] = kc[0]
    out = O.attention(q, kc, vc, 4, 2, 64, pos0)
    v = vc.view(np.float16).astype(np.float64)
    for t in range(T):
        m = v[: pos0 + t + 1].mean(0)
        want = np.concatenate([m[:64], m[:64], m[64:], m[64:]])
        assert np.abs(out[t] - want).max() <= 1e-6
