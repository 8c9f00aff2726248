"""The allocation-free matmul entry point (neko_hip_matmul_noalloc) against neko_hip_matmul.

Both run the same kernels with the same split of K; the allocation-free one keeps its split-K partial
sums (and, for f32 activations, the two f16 planes and their sums) in a fixed device array instead of
the context's workspace. So its outputs must be bit-identical to neko_hip_matmul's on the same inputs,
and -- with integer-valued tables and activations, where every partial sum is exact -- to the
oracle's. Two calls in a row, the second smaller, show that what the first left in the shared array
does not leak into the second. A request that needs more than the array holds is rejected before
anything is launched, and so is a call through a second live context on the same GPU (the array
belongs to the first context that uses it, until that context is destroyed).

The ownership test comes first: it needs the device's array unclaimed, i.e. no earlier
allocation-free call through the thread's shared context (no other test file makes one).
"""
import numpy as np
import pytest
import torch

import mm_tables as M
from nekochat_amd import NekoError, ops
from nekochat_amd._lib import NEKO_ERR_UNSUPPORTED, lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _call(fn, ctx, x, K, tab, fmt, bias, out, flags):
    ctx.bind_torch_stream()
    return fn(ctx.handle, x.data_ptr(), x.stride(0), x.shape[0], K, tab.data_ptr(), tab.shape[1], fmt, tab.shape[0],
              None if bias is None else bias.data_ptr(), out.data_ptr(), out.stride(0), flags, ops.DT_F16 if x.dtype ==
              torch.float16 else ops.DT_F32, ops.DT_F16 if out.dtype == torch.float16 else ops.DT_F32)


def _integer_case(dev, fmt, T, K, N, seed, x_dtype=torch.float16):
    rng = np.random.default_rng(seed)
    tab, _ = M.integer_table(fmt, N, K, rng)
    x = rng.integers(-3, 4, (T, K)).astype(np.float32)
    bias = rng.integers(-20, 21, N).astype(np.float32)
    y0 = rng.integers(-9, 10, (T, N)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev).to(x_dtype)
    return x, tab, bias, y0, xd, torch.from_numpy(tab).to(dev), torch.from_numpy(bias).to(dev)


def test_noalloc_scratch_belongs_to_one_context(dev):
    """Contexts B and C on two torch streams: B's first allocation-free call claims the device's array;
    C's is refused (nothing launched) while its neko_hip_matmul runs from its own workspace; once B is
    destroyed, C's allocation-free calls run and equal neko_hip_matmul's and the oracle's."""
    _case("matmul_noalloc ownership: two contexts on two streams")
    fmt, T, K, N = ops.FMT_FP4, 16, 2560, 6144  # the shared-activation tile kernel with K slices
    x, tab, bias, y0, xd, td, bd = _integer_case(dev, fmt, T, K, N, 650)
    want = O.matmul(fmt, x, tab, K, bias, y0, 0)
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    B, C = ops.Context(dev.index or 0), ops.Context(dev.index or 0)
    try:
        torch.cuda.synchronize()
        outs = {}
        with torch.cuda.stream(s1):
            outs["B"] = torch.from_numpy(y0).to(dev)
            B.check(_call(lib.neko_hip_matmul_noalloc, B, xd, K, td, fmt, bd, outs["B"], 0))
        with torch.cuda.stream(s2):
            outs["C_refused"] = torch.from_numpy(y0).to(dev)
            rc = _call(lib.neko_hip_matmul_noalloc, C, xd, K, td, fmt, bd, outs["C_refused"], 0)
            assert rc == NEKO_ERR_UNSUPPORTED
            msg = lib.neko_hip_last_error(C.handle).decode()
            assert "another live context" in msg, msg
            outs["C_matmul"] = torch.from_numpy(y0).to(dev)
            C.check(_call(lib.neko_hip_matmul, C, xd, K, td, fmt, bd, outs["C_matmul"], 0))
        torch.cuda.synchronize()
        B.close()  # gives up the array
        with torch.cuda.stream(s2):
            outs["C"] = torch.from_numpy(y0).to(dev)
            C.check(_call(lib.neko_hip_matmul_noalloc, C, xd, K, td, fmt, bd, outs["C"], 0))
        torch.cuda.synchronize()
        got = {k: v.cpu().numpy() for k, v in outs.items()}
        assert np.array_equal(got["C_refused"], y0), "a refused call wrote its output"
        for k in ("B", "C_matmul", "C"):
            assert np.array_equal(got[k].view(np.uint32), want.view(np.uint32)), f"{k} differs from the oracle"
    finally:
        B.close()
        C.close()


# (fmt, T, K, N, flags): each takes a split of K -- FP4 / FP8 below 48 tokens the shared-activation
# tile kernel with K slices, F16 from 33 tokens the GEMM with K slices -- and the second of each pair
# is smaller than the first.
PAIRS = [
    ((ops.FMT_FP4, 16, 2560, 6144, 0), (ops.FMT_FP4, 9, 2560, 2560, ops.MM_ACCUMULATE)),
    ((ops.FMT_F16, 64, 2560, 2560, 0), (ops.FMT_F16, 40, 1024, 1024, ops.MM_GELU)),
    ((ops.FMT_FP8, 40, 4096, 2560, ops.MM_ACCUMULATE), (ops.FMT_FP8, 20, 2048, 1024, 0)),
]


@pytest.mark.parametrize("pair", range(len(PAIRS)))
def test_noalloc_matches_matmul(dev, pair):
    ctx = ops.context(dev.index)
    for i, (fmt, T, K, N, flags) in enumerate(PAIRS[pair]):
        _case(f"matmul_noalloc call {i + 1}: fmt={fmt} T={T} K={K} N={N} flags={flags}")
        rng = np.random.default_rng(700 + 10 * pair + i)
        tab, _ = M.integer_table(fmt, N, K, rng)
        x = rng.integers(-3, 4, (T, K)).astype(np.float32)
        bias = rng.integers(-20, 21, N).astype(np.float32)
        y0 = rng.integers(-9, 10, (T, N)).astype(np.float32)
        xd, td, bd = torch.from_numpy(x).to(dev).half(), torch.from_numpy(tab).to(dev), torch.from_numpy(bias).to(dev)
        want = O.matmul(fmt, x, tab, K, bias, y0, flags)
        outs = []
        for fn in (lib.neko_hip_matmul_noalloc, lib.neko_hip_matmul):
            out = torch.from_numpy(y0).to(dev)
            ctx.check(_call(fn, ctx, xd, K, td, fmt, bd, out, flags))
            outs.append(out.cpu().numpy())
        torch.cuda.synchronize()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "noalloc differs from neko_hip_matmul"
        if flags & ops.MM_GELU:  # device GELU vs libm tanh: within 2 f32 ulp of the same argument
            d = np.abs(outs[0].view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
            assert d.max() <= 2, int(d.max())
        else:
            assert np.array_equal(outs[0].view(np.uint32), want.view(np.uint32)), "noalloc differs from the oracle"


# f32 activations past the f32 GEMV's token range: two f16 planes through the MFMA kernels, with the
# planes and sums in the fixed array. (fmt, T, K, N): weights above 2^24 elements split from 9 tokens,
# smaller ones from 17; the third also splits K in the planes' GEMM (partials after the planes).
F32_CASES = [(ops.FMT_FP8, 12, 2560, 19456), (ops.FMT_F16, 24, 2560, 2560), (ops.FMT_FP4, 64, 4096, 2560)]


@pytest.mark.parametrize("case", range(len(F32_CASES)))
def test_noalloc_f32_activations_match_matmul(dev, case):
    fmt, T, K, N = F32_CASES[case]
    _case(f"matmul_noalloc f32 activations: fmt={fmt} T={T} K={K} N={N}")
    ctx = ops.context(dev.index)
    x, tab, bias, y0, xd, td, bd = _integer_case(dev, fmt, T, K, N, 810 + case, torch.float32)
    want = O.matmul(fmt, x, tab, K, bias, y0, ops.MM_ACCUMULATE)
    outs = []
    for fn in (lib.neko_hip_matmul_noalloc, lib.neko_hip_matmul):
        out = torch.from_numpy(y0).to(dev)
        ctx.check(_call(fn, ctx, xd, K, td, fmt, bd, out, ops.MM_ACCUMULATE))
        outs.append(out.cpu().numpy())
    torch.cuda.synchronize()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "noalloc differs from neko_hip_matmul"
    assert np.array_equal(outs[0].view(np.uint32), want.view(np.uint32)), "noalloc differs from the oracle"


def test_noalloc_rejects_f32_planes_beyond_its_array(dev):
    """f32 activations at a prefill size (2048 tokens x K 2560 x N 9728): 101 MB of f16 planes and f32
    sums -- more than the fixed array; nothing is launched."""
    _case("matmul_noalloc oversize f32 planes T=2048 K=2560 N=9728")
    ctx = ops.context(dev.index)
    K, N, T = 2560, 9728, 2048
    tab = torch.zeros((N, M.row_bytes(ops.FMT_F16, K)), dtype=torch.uint8, device=dev)
    x = torch.zeros((T, K), dtype=torch.float32, device=dev)
    out = torch.full((T, N), 7.0, dtype=torch.float32, device=dev)
    rc = _call(lib.neko_hip_matmul_noalloc, ctx, x, K, tab, ops.FMT_F16, None, out, 0)
    assert rc == NEKO_ERR_UNSUPPORTED
    msg = lib.neko_hip_last_error(ctx.handle).decode()
    assert "f16 planes" in msg and "at most" in msg, msg
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_noalloc_rejects_split_beyond_its_array(dev):
    """FP8 rows, 47 tokens x 151936 rows (a Qwen3 tied LM head): the tile kernel splits K = 2048 four
    ways, 114 MB of partial sums -- more than the fixed array; nothing is launched."""
    _case("matmul_noalloc oversize FP8 T=47 K=2048 N=151936")
    ctx = ops.context(dev.index)
    K, N, T = 2048, 151936, 47
    tab = torch.zeros((N, M.row_bytes(ops.FMT_FP8, K)), dtype=torch.uint8, device=dev)
    x = torch.zeros((T, K), dtype=torch.float16, device=dev)
    out = torch.full((T, N), 7.0, dtype=torch.float32, device=dev)
    rc = _call(lib.neko_hip_matmul_noalloc, ctx, x, K, tab, ops.FMT_FP8, None, out, 0)
    assert rc == NEKO_ERR_UNSUPPORTED
    msg = lib.neko_hip_last_error(ctx.handle).decode()
    assert "allocation-free" in msg and "partial sums" in msg, msg
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    with pytest.raises(NekoError):
        ctx.check(rc)
