"""The allocation-free matmul entry point (neko_hip_matmul_noalloc) against neko_hip_matmul.

Both run the same kernels with the same split of K; the allocation-free one keeps its split-K partial
sums in a fixed device array instead of the context's workspace. So its outputs must be bit-identical
to neko_hip_matmul's on the same inputs, and -- with integer-valued tables and activations, where every
partial sum is exact -- to the oracle's. Two calls in a row, the second smaller, show that what the
first left in the shared array does not leak into the second. A split that needs more than the array
holds is rejected before anything is launched.
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
    assert "allocation-free" in msg and "at most" in msg, msg
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    with pytest.raises(NekoError):
        ctx.check(rc)
