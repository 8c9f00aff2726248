"""GPU parity of the weight matmul (neko_hip_matmul) against the oracle and exact arithmetic.

The reference sums each dot product sequentially in f32 on the CPU and in a reduction tree on its
GPU, so no summation order is canonical. The bars:
  - integer-valued weights (codes times power-of-two scales) and activations: every partial sum is
    exact, so outputs are bit-identical to the oracle in any order -- a dropped, repeated or
    misplaced term, a wrong scale or a wrong token/row mapping changes the bits;
  - random data: |y - exact| <= (K + 64) * 2^-24 * (sum_k |x_k w_k| + |bias|) against the float64
    product of the oracle's dequantised weights (the worst-case bound of an f32 sum of K exact
    products in any order, with the per-block scale, cross-wave and bias additions); the observed
    error is reported and is a few units of 2^-24 * that magnitude.
"""
import numpy as np
import pytest
import torch

import mm_tables as M
from nekochat_amd import NekoError, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
FMTS = [ops.FMT_F16, ops.FMT_FP8, ops.FMT_FP4]


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _bound_check(got, exact, mag, K, what):
    err = np.abs(got.astype(np.float64) - exact)
    ratio = float((err / np.maximum(mag * U, 1e-300)).max())
    print(f"[parity] {what}: max |y - exact| = {ratio:.2f} * 2^-24 * sum|x w| (bound {K + 64})", flush=True)
    assert (err <= (K + 64) * U * mag + 1e-30).all(), f"{what}: error beyond the f32 summation bound"


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 16, 17, 64, 100, 128, 300])
def test_matmul_integer_rows_bitexact(dev, fmt, T):
    """K = 320 (ten 32-blocks: two 4-block groups and a 2-block tail), N = 37 (a partial row tile).
    T <= 2: the GEMV; 3..47: the MFMA tile kernels (F16: up to 32); above: the GEMM (300: a partial
    token tile)."""
    _case(f"matmul integer fmt={fmt} T={T}")
    rng = np.random.default_rng(100 + 10 * fmt + T)
    K, N = 320, 37
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev).half()
    td = torch.from_numpy(tab).to(dev)
    bd = torch.from_numpy(bias).to(dev)
    for flags, b in ((0, None), (0, bias), (ops.MM_ACCUMULATE, bias), (ops.MM_GELU, bias),
                     (ops.MM_GELU | ops.MM_ACCUMULATE, None)):
        want = O.matmul(fmt, x, tab, K, b, y0, flags)
        out = torch.from_numpy(y0).to(dev)
        ops.matmul(xd, td, fmt, K, bias=None if b is None else bd, out=out, flags=flags)
        got = out.cpu().numpy()
        if flags & ops.MM_GELU:  # device GELU vs libm tanh: within 2 f32 ulp of the same argument
            d = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
            assert d.max() <= 2, (flags, int(d.max()))
        else:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (flags, b is None)
    # f16 output: one rounding of the exact value
    out16 = ops.matmul(xd, td, fmt, K, bias=bd, out_dtype=torch.float16)
    want16 = O.f32_to_f16(O.matmul(fmt, x, tab, K, bias))
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), want16)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K", [2048, 2080])
def test_matmul_split_k_integer_bitexact(dev, fmt, K):
    """A long K over few output tiles (T = 130, N = 37: two tiles) runs as K slices whose partial
    sums are reduced afterwards; with integer values every partial is exact, so the result is.
    K = 2048 takes the 64-deep GEMM (K % 64 == 0), K = 2080 the 32-deep one (K % 64 == 32): two
    tiles x 8 slices each, then the ordered reduction, with and without accumulation."""
    rng = np.random.default_rng(400 + fmt + K)
    T, N = 130, 37
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    for flags in (0, ops.MM_ACCUMULATE):
        _case(f"matmul split-K integer fmt={fmt} K={K} flags={flags}")
        out = torch.from_numpy(y0).to(dev)
        ops.matmul(torch.from_numpy(x).to(dev).half(), torch.from_numpy(tab).to(dev), fmt, K,
                   bias=torch.from_numpy(bias).to(dev), out=out, flags=flags)
        want = O.matmul(fmt, x, tab, K, bias, y0, flags)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), flags


def test_matmul_split_k_graph_replays(dev):
    """A split-K matmul captured in a HIP graph (after one uncaptured call at its shape, so the
    context's workspace is already large enough) replays bit-identically to an uncaptured call, on
    fresh inputs each replay with eager work and synchronisations in between."""
    _case("matmul split-K graph capture + 3 replays")
    rng = np.random.default_rng(950)
    fmt, T, K, N = ops.FMT_FP4, 16, 2560, 6144
    tab, _ = M.integer_table(fmt, N, K, rng)
    td = torch.from_numpy(tab).to(dev)
    xd = torch.from_numpy(rng.integers(-4, 5, (T, K)).astype(np.float32)).to(dev).half()
    out_g = torch.zeros((T, N), dtype=torch.float32, device=dev)
    ops.matmul(xd, td, fmt, K, out=out_g)  # warm-up: sizes the workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.matmul(xd, td, fmt, K, out=out_g)
    for i in range(3):
        xd.copy_(torch.from_numpy(rng.integers(-4, 5, (T, K)).astype(np.float32)).half())
        g.replay()
        torch.cuda.synchronize()
        eager = ops.matmul(xd, td, fmt, K)
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int32), eager.view(torch.int32)), f"replay {i}"


def test_matmul_f16_prefill_graph_replays(dev):
    """An F16 product at prefill size captured in a HIP graph runs on the own kernels (the hipBLASLt
    path is not taken under capture: its stream-K kernels clear their flags with a memset), and each of
    three replays on fresh integer-valued inputs, with eager work and synchronisations between them,
    equals the uncaptured call (hipBLASLt) bit for bit: every partial sum is exact."""
    _case("matmul F16 prefill graph capture + 3 replays")
    rng = np.random.default_rng(951)
    fmt, T, K, N = ops.FMT_F16, 2048, 1024, 4096
    tab, _ = M.integer_table(fmt, N, K, rng)
    td = torch.from_numpy(tab).to(dev)
    xd = torch.from_numpy(rng.integers(-4, 5, (T, K)).astype(np.float32)).to(dev).half()
    out_g = torch.zeros((T, N), dtype=torch.float32, device=dev)
    ops.matmul(xd, td, fmt, K, out=out_g)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.matmul(xd, td, fmt, K, out=out_g)
    for i in range(3):
        xd.copy_(torch.from_numpy(rng.integers(-4, 5, (T, K)).astype(np.float32)).half())
        g.replay()
        torch.cuda.synchronize()
        eager = ops.matmul(xd, td, fmt, K)
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int32), eager.view(torch.int32)), f"replay {i}"


def test_matmul_workspace_growth_refused_under_capture(dev):
    """A fresh context has no workspace: a split-K call captured into a graph would have to allocate
    it, and fails with NEKO_ERR_INVALID instead (naming the way out) without breaking the capture."""
    _case("matmul workspace growth under capture")
    from nekochat_amd._lib import NEKO_ERR_INVALID, lib
    ctx = ops.Context(dev.index)
    rng = np.random.default_rng(951)
    fmt, T, K, N = ops.FMT_FP4, 16, 2560, 6144
    tab, _ = M.integer_table(fmt, N, K, rng)
    td = torch.from_numpy(tab).to(dev)
    xd = torch.from_numpy(rng.integers(-4, 5, (T, K)).astype(np.float32)).to(dev).half()
    out = torch.zeros((T, N), dtype=torch.float32, device=dev)
    side = torch.zeros(4, device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        assert lib.neko_hip_set_stream(ctx.handle, s) == 0
        rc = lib.neko_hip_matmul(ctx.handle, xd.data_ptr(), K, T, K, td.data_ptr(), td.shape[1], fmt, N, None,
                                 out.data_ptr(), N, 0, ops.DT_F16, ops.DT_F32)
        side.add_(1.0)
    msg = lib.neko_hip_last_error(ctx.handle).decode()
    assert rc == NEKO_ERR_INVALID and "captured" in msg, (rc, msg)
    g.replay()
    torch.cuda.synchronize()
    assert bool((side == 1.0).all()) and bool((out == 0).all())
    assert lib.neko_hip_set_stream(ctx.handle, None) == 0
    ctx.close()


def test_matmul_split_k_across_stream_switch(dev):
    """Split-K calls share the context's f32 workspace. Calls issued alternately on two torch
    streams (each switch re-routes the context; the later shapes grow the workspace) stay ordered:
    every output equals the exact integer product."""
    _case("matmul split-K across stream switches")
    rng = np.random.default_rng(900)
    cases = []
    for T, K, N in ((16, 4096, 2560), (16, 2560, 6144), (40, 9728, 2560)):  # all split K
        tab, w = M.integer_table(ops.FMT_FP4, N, K, rng)
        x = rng.integers(-4, 5, (T, K)).astype(np.float32)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.abs(exact).max() < 2 ** 24
        cases.append((torch.from_numpy(x.astype(np.float16)).to(dev), torch.from_numpy(tab).to(dev), K,
                      exact.astype(np.float32)))
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(dev), torch.cuda.Stream(dev))
    outs = []
    for rep in range(2):
        for i, (xd, td, K, _) in enumerate(cases):
            with torch.cuda.stream(streams[(i + rep) % 2]):
                outs.append((i, ops.matmul(xd, td, ops.FMT_FP4, K)))
    torch.cuda.synchronize()
    for i, y in outs:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), cases[i][3].view(np.uint32)), i


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,N", [
    (2000, 320, 8200),  # FP8 / FP4: 256-token x 128-row tiles (enough to fill the GPU), partial in both
    (4000, 320, 8200),  # 256 x 256 tiles, direct-to-LDS loads (two per CU; FP8 / FP4 decoded per wave), partial in both
    (4000, 320, 4100),  # F16: 128 x 128 tiles (too few 256 x 256 tiles for two per CU), partial in both
    (300, 352, 37),     # K % 64 == 32: the 32-wide staged kernel
    (200, 320, 37),     # 128 x 128 tiles in 64-wide stages
    (20, 4096, 100),    # 20 tokens: activations staged per K slice, several slices reduced in order
    (47, 2080, 300),    # three token tiles, K slices ending in a partial group
    (12, 2560, 700),    # 12 tokens: F16 / FP8 per-wave tiles, FP4 staged per K slice (several slices)
])
def test_matmul_gemm_tilings_integer_bitexact(dev, fmt, T, K, N):
    """Integer-valued weights and activations through each MFMA tiling: every partial sum is exact,
    so y = bias + x . w (+ y0 with accumulate) is bit-identical to the float64 product rounded once."""
    _case(f"matmul GEMM tiling integer fmt={fmt} T={T} K={K} N={N}")
    rng = np.random.default_rng(500 + fmt + T + K)
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert np.abs(exact).max() < 2 ** 24
    xd, td, bd = (torch.from_numpy(v).to(dev) for v in (x.astype(np.float16), tab, bias))
    got = ops.matmul(xd, td, fmt, K, bias=bd).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), exact.astype(np.float32).view(np.uint32))
    out = torch.from_numpy(y0).to(dev)
    ops.matmul(xd, td, fmt, K, bias=bd, out=out, flags=ops.MM_ACCUMULATE)
    want = (y0.astype(np.float64) + exact).astype(np.float32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,N", [
    (4096, 64, 8192),   # 256 x 256 tiles (two per CU), direct-to-LDS loads
    (4096, 64, 4100),   # F16: 128 x 128 tiles; FP8 / FP4: 256-token x 128-row tiles; a 4-column last tile
])
def test_matmul_gemm_epilogue_variants(dev, fmt, T, K, N):
    """The GEMM kernels' regrouped epilogue in each of its forms, on integer-valued data (the sums are
    exact): bias + GELU (the separately instantiated GELU epilogue; checked on a random sample of
    outputs against the oracle's GELU of the same exact argument, within 2 f32 ulp), f16 output (one
    rounding of the exact value, every output), and an output slice that starts one float into each row
    with an odd row stride (no 4-wide stores: the element-wise tail path), accumulated into, with the
    columns either side left untouched."""
    _case(f"matmul GEMM epilogues fmt={fmt} T={T} K={K} N={N}")
    rng = np.random.default_rng(700 + fmt + N)
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert np.abs(exact).max() < 2 ** 24
    e32 = exact.astype(np.float32)
    xd, td, bd = (torch.from_numpy(v).to(dev) for v in (x.astype(np.float16), tab, bias))

    got = ops.matmul(xd, td, fmt, K, bias=bd, flags=ops.MM_GELU).cpu().numpy()
    idx = rng.integers(0, T * N, 200_000)
    idx = np.concatenate([idx, np.arange(T * N - N, T * N)])  # and the whole last row
    want = np.array([O.lib().oracle_gelu(float(v)) for v in e32.ravel()[idx]], np.float32)
    d = np.abs(got.ravel()[idx].view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert d.max() <= 2, int(d.max())

    got16 = ops.matmul(xd, td, fmt, K, bias=bd, out_dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), O.f32_to_f16(e32))

    base = rng.standard_normal((T, N + 3)).astype(np.float32)
    buf = torch.from_numpy(base).to(dev)
    ops.matmul(xd, td, fmt, K, bias=bd, out=buf[:, 1:1 + N], flags=ops.MM_ACCUMULATE)
    res = buf.cpu().numpy()
    want = (base[:, 1:1 + N].astype(np.float64) + exact).astype(np.float32)
    assert np.array_equal(res[:, 1:1 + N].view(np.uint32), want.view(np.uint32))
    assert np.array_equal(res[:, :1], base[:, :1]) and np.array_equal(res[:, 1 + N:], base[:, 1 + N:])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,N", [
    (1, 2560, 6144),    # Qwen3-4B decode: q/k/v projection
    (1, 9728, 2560),    # Qwen3-4B decode: down projection
    (8, 2560, 19456),   # Qwen3-4B batch-8 decode: gate/up projection
    (16, 2560, 6144),   # Qwen3-4B batch-16 decode: q/k/v projection
    (33, 4096, 2560),   # o projection, three token tiles
    (3, 32, 40),        # one block
    (200, 768, 96),     # GPT-2 width, several token chunks
    (2, 4096, 2560),    # two-token decode
    (2, 20480, 64),     # two tokens whose activations exceed the GEMV's LDS stage: two token chunks
    (4, 9728, 64),      # four tokens, long K: MFMA tiles
    (4, 768, 3072),     # GPT-2 MLP, four tokens
    (256, 2560, 6144),  # prefill chunk: GEMM tiles
    (300, 1024, 700),   # partial token and row tiles
    (512, 9728, 2560),  # down projection, long K
    (512, 2560, 16384), # FP8 / FP4: 256-token x 128-row tiles
    (2048, 1024, 16384),  # 256 x 256 tiles with direct-to-LDS loads (FP8 / FP4: codes and scales too)
    (4096, 1024, 4096),   # F16: 128 x 128 tiles, two stages of register prefetch
    (47, 9728, 2560),   # three token tiles, activations staged per K slice, slices reduced in order
])
def test_matmul_random_within_bound(dev, fmt, T, K, N):
    _case(f"matmul random fmt={fmt} T={T} K={K} N={N}")
    rng = np.random.default_rng(7 * T + K + N + fmt)
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    tab, used = ops.quantize_rows(fmt, w)
    assert used == fmt
    wd = M.dequant(fmt, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    y = ops.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(tab).to(dev), fmt, K,
                   bias=torch.from_numpy(bias).to(dev)).cpu().numpy()
    exact, mag = M.exact_and_bound(x.astype(np.float32), wd, bias)
    _bound_check(y, exact, mag, K, f"fmt={fmt} T={T} K={K} N={N}")
    if T * N <= 4096:
        want = O.matmul(fmt, x.astype(np.float32), tab, K, bias)
        assert np.abs(y - want).max() <= float(((2 * K + 65) * U * mag).max())


@pytest.mark.parametrize("T,K,N", [
    (2048, 1024, 16384),  # 256 x 256 tiles on the own kernels
    (4096, 1024, 4096),   # 128 x 128 tiles on the own kernels
    (2048, 2560, 2560),   # an o-projection-shaped product
    (512, 9728, 2560),    # the down projection at the library's threshold
    (64, 2560, 19456),    # gate/up-wide rows: the library from 64 tokens
])
def test_matmul_f16_prefill_library_and_own(dev, T, K, N):
    """Plain F16 products from 512 tokens run on hipBLASLt by default and on the library's own MFMA
    kernels with the context's switch off (neko_hip_set_matmul_library): both bit-identical to the exact
    result on integer-valued data -- f32 output with bias, f16 output (one rounding of the exact value)
    and accumulation into y -- and both within the f32 summation bound on random data."""
    ctx = ops.context(dev.index or 0)
    rng = np.random.default_rng(900 + T + N)
    tab, w = M.integer_table(ops.FMT_F16, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert np.abs(exact).max() < 2 ** 24
    e32 = exact.astype(np.float32)
    xd, td, bd = (torch.from_numpy(v).to(dev) for v in (x.astype(np.float16), tab, bias))
    y0 = rng.integers(-1000, 1001, (T, N)).astype(np.float32)
    wr = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    tr, _ = ops.quantize_rows(ops.FMT_F16, wr)
    xr = rng.standard_normal((T, K)).astype(np.float16)
    br = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ex_r, mag = M.exact_and_bound(xr.astype(np.float32), M.dequant(ops.FMT_F16, tr, K), br)
    for lib in (True, False):
        _case(f"matmul F16 prefill {'hipBLASLt' if lib else 'own kernels'} T={T} K={K} N={N}")
        ctx.set_matmul_library(lib)
        try:
            got = ops.matmul(xd, td, ops.FMT_F16, K, bias=bd).cpu().numpy()
            assert np.array_equal(got.view(np.uint32), e32.view(np.uint32))
            got16 = ops.matmul(xd, td, ops.FMT_F16, K, bias=bd, out_dtype=torch.float16).cpu().numpy()
            assert np.array_equal(got16.view(np.uint16), O.f32_to_f16(e32))
            # accumulated without a bias (the library's), and with one (y + (dot + bias), own kernels)
            acc = torch.from_numpy(y0).to(dev)
            ops.matmul(xd, td, ops.FMT_F16, K, out=acc, flags=ops.MM_ACCUMULATE)
            want = (y0.astype(np.float64) + (exact - bias)).astype(np.float32)
            assert np.array_equal(acc.cpu().numpy().view(np.uint32), want.view(np.uint32))
            acc = torch.from_numpy(y0 + 0.25).to(dev)
            ops.matmul(xd, td, ops.FMT_F16, K, bias=bd, out=acc, flags=ops.MM_ACCUMULATE)
            want = ((y0 + 0.25).astype(np.float64) + exact).astype(np.float32)
            assert np.array_equal(acc.cpu().numpy().view(np.uint32), want.view(np.uint32))
            yr = ops.matmul(torch.from_numpy(xr).to(dev), torch.from_numpy(tr).to(dev), ops.FMT_F16, K,
                            bias=torch.from_numpy(br).to(dev)).cpu().numpy()
            _bound_check(yr, ex_r, mag, K, f"F16 {'hipBLASLt' if lib else 'own'} T={T} K={K} N={N}")
        finally:
            ctx.set_matmul_library(True)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8, 9, 16, 17, 33])
def test_matmul_f32_activations_integer_bitexact(dev, fmt, T):
    """f32 activations -- the reference's own type, as the ComputeBackend adapter passes them: up to 8
    tokens the GEMV's f32 form (passes of 1, 2 or 4 tokens; up to 16 for weights of at most 2^24
    elements, as here), from 9 (17) two f16 planes (each row scaled by a power of two) through the
    MFMA kernels and an exact rescale. Integer-valued data, every flag, bit-identical to the oracle;
    f16 output one rounding of the exact value."""
    _case(f"matmul f32 activations integer fmt={fmt} T={T}")
    rng = np.random.default_rng(900 + 10 * fmt + T)
    K, N = 320, 37
    tab, w = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-4, 5, (T, K)).astype(np.float32)
    bias = rng.integers(-50, 51, N).astype(np.float32)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    td = torch.from_numpy(tab).to(dev)
    bd = torch.from_numpy(bias).to(dev)
    for flags, b in ((0, None), (0, bias), (ops.MM_ACCUMULATE, bias), (ops.MM_GELU, bias)):
        want = O.matmul(fmt, x, tab, K, b, y0, flags)
        out = torch.from_numpy(y0).to(dev)
        ops.matmul(xd, td, fmt, K, bias=None if b is None else bd, out=out, flags=flags)
        got = out.cpu().numpy()
        if flags & ops.MM_GELU:
            d = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
            assert d.max() <= 2, (flags, int(d.max()))
        else:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (flags, b is None)
    out16 = ops.matmul(xd, td, fmt, K, bias=bd, out_dtype=torch.float16)
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), O.f32_to_f16(O.matmul(fmt, x, tab, K, bias)))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,K,N", [
    (1, 2560, 6144),    # Qwen3-4B decode through the adapter: q/k/v
    (1, 9728, 2560),    # down: one token per pass (39 KB of f32 activations in LDS)
    (4, 2560, 19456),   # four tokens per pass
    (4, 4096, 2560),    # two passes of two tokens (64 KB of LDS holds two f32 rows of 4096)
    (2, 20480, 64),     # f32 activations too long for the GEMV's LDS: the generic kernel
    (8, 2560, 19456),   # two passes of four tokens
    (12, 2560, 19456),  # from 9 tokens: two f16 planes through the MFMA tile kernels
    (64, 2560, 6144),   # ... the GEMM
    (300, 1024, 700),   # ... partial token and row tiles
    (512, 9728, 2560),  # ... long K
])
def test_matmul_f32_activations_random_within_bound(dev, fmt, T, K, N):
    _case(f"matmul f32 activations random fmt={fmt} T={T} K={K} N={N}")
    rng = np.random.default_rng(11 * T + K + N + fmt)
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    tab, used = ops.quantize_rows(fmt, w)
    wd = M.dequant(fmt, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    y = ops.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(tab).to(dev), fmt, K,
                   bias=torch.from_numpy(bias).to(dev)).cpu().numpy()
    exact, mag = M.exact_and_bound(x, wd, bias)
    _bound_check(y, exact, mag, K, f"f32 x fmt={fmt} T={T} K={K} N={N}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [16, 24])
def test_matmul_f32_activations_row_magnitudes(dev, fmt, T):
    """f32 activation rows far outside f16's range, tiny, zero, and with values 2^30 apart in one row:
    T = 24 through the two-plane path (each row scaled by its own power of two, the 3e-38 row at the
    scale's 2^126 clamp), T = 16 through the f32 GEMV (weights of at most 2^24 elements keep it through
    16 tokens): within the bound."""
    _case(f"matmul f32 activations row magnitudes fmt={fmt} T={T}")
    rng = np.random.default_rng(77 + fmt)
    K, N = 2560, 384
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    tab, _ = ops.quantize_rows(fmt, w)
    wd = M.dequant(fmt, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    scale = np.array([1e30, 1e-30, 1e5, 1e-5, 0.0, 7e4, 1.0, 3e-38] + [1.0] * (T - 8), np.float32)
    x *= scale[:, None]
    x[8, :K // 2] *= np.float32(2.0 ** -30)  # one row holding values 2^30 apart
    x[9, 7] = np.float32(6e4)                # one outlier in an ordinary row
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    y = ops.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(tab).to(dev), fmt, K,
                   bias=torch.from_numpy(bias).to(dev)).cpu().numpy()
    exact, mag = M.exact_and_bound(x, wd, bias)
    assert np.isfinite(y).all()
    _bound_check(y, exact, mag, K, f"f32 row magnitudes fmt={fmt}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T", [4, 24])
def test_matmul_f32_activations_nonfinite(dev, fmt, T):
    """f32 activation rows holding one +inf, one -inf or one NaN (T = 4: the f32 GEMV; T = 24: the
    two-plane split, where such a value must not set its row's scale): every output of those rows is
    the IEEE value of the float64 product -- +-inf by the sign of the weight, NaN where the weight is
    zero or the value is NaN -- and every other row stays within the bound."""
    _case(f"matmul f32 activations non-finite fmt={fmt} T={T}")
    rng = np.random.default_rng(91 + 7 * fmt + T)
    K, N = 2560, 384
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    tab, _ = ops.quantize_rows(fmt, w)
    wd = M.dequant(fmt, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    special = {0: (5, np.inf), 1: (700, -np.inf), 2: (1300, np.nan)}
    for t, (k, v) in special.items():
        x[t, k] = v
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    y = ops.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(tab).to(dev), fmt, K,
                   bias=torch.from_numpy(bias).to(dev)).cpu().numpy()
    wz = wd.astype(np.float64)
    for t, (k, v) in special.items():
        col = wz[:, k]
        if np.isnan(v):
            want_inf = np.zeros(N, bool)
        else:
            want_inf = col != 0
            assert np.array_equal(np.sign(y[t][want_inf]), np.sign(v * col[want_inf])), f"row {t}: signs"
        assert np.array_equal(np.isinf(y[t]), want_inf), f"row {t}: infinities"
        assert np.array_equal(np.isnan(y[t]), ~want_inf), f"row {t}: NaNs"
    rest = np.arange(3, T)
    exact, mag = M.exact_and_bound(x[rest], wd, bias)
    _bound_check(y[rest], exact, mag, K, f"f32 non-finite rows fmt={fmt} T={T}: the other rows")


def test_matmul_generic_paths(dev):
    """f32 activations, misaligned rows, K not a multiple of 32 (F16 only), f16 output."""
    _case("matmul generic paths")
    rng = np.random.default_rng(5)
    for fmt, K, xdt, off in ((ops.FMT_F16, 100, torch.float32, 0), (ops.FMT_FP8, 256, torch.float32, 3),
                             (ops.FMT_FP4, 96, torch.float16, 3), (ops.FMT_F16, 64, torch.float16, 1)):
        T, N = 6, 21
        w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
        tab, used = ops.quantize_rows(fmt, w)
        wd = M.dequant(used, tab, K)
        buf = torch.from_numpy(rng.standard_normal((T, K + 8)).astype(np.float32)).to(dev).to(xdt)
        x = buf[:, off:off + K]
        xh = x.float().cpu().numpy()
        for ydt in (torch.float32, torch.float16):
            y = ops.matmul(x, torch.from_numpy(tab).to(dev), used, K, out_dtype=ydt).float().cpu().numpy()
            exact, mag = M.exact_and_bound(xh, wd)
            if ydt == torch.float32:
                _bound_check(y, exact, mag, K, f"generic fmt={used} K={K} x={xdt}")
            else:
                assert np.abs(y - exact).max() <= np.abs(exact).max() * 2.0 ** -10 + 1e-6


@pytest.mark.parametrize("T", [3, 20])
def test_matmul_accumulate_into_column_slice(dev, T):
    """y is columns [64, 64 + N) of a wider f32 buffer (the shaders' nOffset): bias + GELU added into it;
    the columns outside stay untouched (T = 3: the decode path, T = 20: the tile path)."""
    _case(f"matmul accumulate into a column slice T={T}")
    rng = np.random.default_rng(9 + T)
    K, N = 512, 48
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    tab, _ = ops.quantize_rows(ops.FMT_FP8, w)
    wd = M.dequant(ops.FMT_FP8, tab, K)
    x = rng.standard_normal((T, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    base = rng.standard_normal((T, 256)).astype(np.float32)
    buf = torch.from_numpy(base).to(dev)
    ops.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(tab).to(dev), ops.FMT_FP8, K,
               bias=torch.from_numpy(bias).to(dev), out=buf[:, 64:64 + N], flags=ops.MM_GELU | ops.MM_ACCUMULATE)
    got = buf.cpu().numpy()
    assert np.array_equal(got[:, :64], base[:, :64]) and np.array_equal(got[:, 64 + N:], base[:, 64 + N:])
    exact, mag = M.exact_and_bound(x.astype(np.float32), wd, bias)
    gel = np.array([O.lib().oracle_gelu(float(v)) for v in exact.ravel()], np.float64).reshape(T, N)
    want = base[:, 64:64 + N].astype(np.float64) + gel
    tol = 1.2 * (K + 64) * U * mag + 4 * U * (np.abs(gel) + np.abs(want))
    assert (np.abs(got[:, 64:64 + N] - want) <= tol).all()


def test_matmul_empty_and_invalid(dev):
    _case("matmul empty / invalid")
    x = torch.zeros((4, 64), dtype=torch.float16, device=dev)
    tab = torch.zeros((8, O.lib().oracle_quant_row_bytes(1, 64)), dtype=torch.uint8, device=dev)
    out = ops.matmul(x[:0], tab, ops.FMT_FP8, 64)
    assert out.shape == (0, 8)
    with pytest.raises(NekoError):
        ops.matmul(x, tab, 7, 64)  # bad format
    with pytest.raises(NekoError):
        ops.matmul(x, tab, ops.FMT_FP8, 64, flags=4)  # bad flags
    with pytest.raises(NekoError):
        ops.matmul(x[:, :48], tab, ops.FMT_FP8, 48)  # FP8 rows need K % 32 == 0
    with pytest.raises(NekoError):
        ops.matmul(x, tab, ops.FMT_FP8, 64, out=x.view(torch.float32)[:, :8])  # y overlaps x
    with pytest.raises(NekoError):
        ops.matmul(x, tab[:, :40], ops.FMT_FP8, 64)  # rows shorter than a K=64 FP8 row
