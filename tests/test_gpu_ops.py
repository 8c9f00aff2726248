"""GPU parity of every hot-path op against the oracle, through the C ABI (nekochat_amd.ops).

Bars: embedding gather / dequant bit-exact; norms, activations and RoPE within 2 fp16 ulp of the
oracle (in practice almost every output is bit-identical: the kernels accumulate in double and round
where the reference rounds). Configured shapes run at full size; edge cases cover empty inputs, odd
widths (fallback kernels), strided rows, in-place calls, f32 activations and out-of-range positions.
"""
import numpy as np
import pytest
import torch

from conftest import assert_f16_close, to_bits
from nekochat_amd import NekoError, ops
from nekochat_amd import workloads as wl
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _f16(shape, stream, dev, mean=0.0, std=1.0):
    return wl.normal_f16(shape, mean, std, stream, dev)


def _w(n, stream, dev, mean=1.0, std=0.05):
    return wl.weight_f32(n, mean, std, stream, dev)


# ------------------------------------------------------------------ RMSNorm

@pytest.mark.parametrize("T,C,eps", [
    (64, 1024, 1e-6),      # Qwen3-0.6B decode (one round, one row per wave)
    (8192, 2560, 1e-6),    # Qwen3-4B prefill (one round, two rows per wave)
    (16384, 1536, 1e-5),   # Granite pre-norm (one row per wave over the whole grid)
    (12288, 2560, 1e-6),   # one round, three rows per wave
    (4096, 2560, 1e-6),    # one round, one row of five chunks per lane
    (8191, 2000, 1e-6),    # two rows per wave, the last wave one short; 250 chunks: lanes past the row end
    (32768, 2560, 1e-6),   # one row per wave over the whole grid (more than one round's three rows per wave)
    (3, 96, 1e-6),         # reference self-test width
    (5, 4104, 1e-6),       # four waves per row
    (7, 100, 1e-6),        # width not a multiple of 8: fallback kernel
    (2, 20000, 1e-6),      # wider than the register path
    (1, 8, 1e-6),
])
def test_rmsnorm_f16(dev, T, C, eps):
    _case(f"rmsnorm f16 T={T} C={C}")
    x = _f16((T, C), 1, dev)
    w = _w(C, 2, dev)
    y = ops.rms_norm(x, w, eps)
    want = O.rmsnorm_f16(to_bits(x), w.cpu().numpy(), eps)
    d = assert_f16_close(to_bits(y), want, what=f"rmsnorm {T}x{C}")
    assert np.count_nonzero(d) <= max(2, d.size // 10000), "more outputs off the reference than double accumulation allows"


def test_rmsnorm_strided_inplace_and_edges(dev):
    _case("rmsnorm strided / in place / empty / zero rows")
    T, C, S = 33, 1024, 1536
    buf = _f16((T, S), 3, dev)
    buf[5].zero_()  # zero row: scale = 1/sqrt(eps)
    buf[6].fill_(0.5)  # constant row
    x = buf[:, :C]
    w = _w(C, 4, dev)
    want = O.rmsnorm_f16(to_bits(x), w.cpu().numpy(), 1e-6)
    tail = to_bits(buf[:, C:]).copy()
    ops.rms_norm(x, w, 1e-6, out=x)  # in place on a strided view
    assert_f16_close(to_bits(x), want, what="rmsnorm in place strided")
    assert np.array_equal(to_bits(buf[:, C:]), tail), "columns past C were written"
    empty = torch.empty((0, C), dtype=torch.float16, device=dev)
    assert ops.rms_norm(empty, w, 1e-6).shape == (0, C)


def test_prepared_call_keeps_its_stream(dev):
    """ops.prepare replays one C call on the torch stream current at preparation, also after another
    op has routed the thread's context to a different stream; its output equals a direct call's."""
    _case("prepared rms_norm replay after a stream switch")
    x, w = _f16((64, 1024), 11, dev), _w(1024, 12, dev)
    want = ops.rms_norm(x, w, 1e-6)
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    out = torch.empty_like(x)
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        run, res = ops.prepare(ops.rms_norm, x, w, 1e-6, out=out)
    assert res is out
    with torch.cuda.stream(s2):
        ops.rms_norm(_f16((8, 1024), 13, dev), w, 1e-6)  # routes the context to s2
    ctx = ops.context(dev.index if dev.index is not None else 0)
    assert ctx._bound == s2.cuda_stream
    out.zero_()
    torch.cuda.synchronize()
    run()
    assert ctx._bound == s1.cuda_stream
    s1.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("T", [17, 40000, 8192])
def test_rmsnorm_f32(dev, T):
    """17 rows of 2560 floats: four waves per row; 40000 rows of 1024 floats: the one-row-per-wave
    grid; 8192 rows of 1024: one round, two rows per wave."""
    _case(f"rmsnorm f32 T={T}")
    C = 2560 if T == 17 else 1024
    x = _f16((T, C), 5, dev).float() * 20
    w = _w(C, 6, dev)
    y = ops.rms_norm(x, w, 1e-6)
    want = np.empty((T, C), np.float32)
    O.lib().oracle_rmsnorm(O._ptr(x.cpu().numpy()), O._ptr(want), O._ptr(w.cpu().numpy()), T, C, 1e-6)
    np.testing.assert_allclose(y.cpu().numpy(), want, rtol=2e-7, atol=0)


# ------------------------------------------------------------------ LayerNorm

@pytest.mark.parametrize("T,C,shift", [(128, 768, 0.0), (64, 1024, 100.0), (3, 96, 0.0), (9, 770, 3.0), (4, 2560, 0.0),
                                       (8192, 768, 2.0), (12287, 512, 0.5),  # one round: two / three rows per wave
                                       (40000, 768, 1.0)])  # the last: one row per wave over the grid
def test_layernorm_f16(dev, T, C, shift):
    _case(f"layernorm f16 T={T} C={C} shift={shift}")
    x = _f16((T, C), 7, dev, mean=shift)
    g = _w(C, 8, dev, 1.0, 0.02)
    b = _w(C, 9, dev, 0.0, 0.02)
    y = ops.layer_norm(x, g, b, 1e-5)
    want = O.layernorm_f16(to_bits(x), g.cpu().numpy(), b.cpu().numpy(), 1e-5)
    assert_f16_close(to_bits(y), want, what=f"layernorm {T}x{C}")


def test_layernorm_constant_row(dev):
    _case("layernorm constant rows")
    x = torch.full((4, 768), 1.5, dtype=torch.float16, device=dev)
    g = _w(768, 10, dev)
    b = _w(768, 11, dev, 0.0, 0.02)
    y = ops.layer_norm(x, g, b, 1e-5)
    want = O.layernorm_f16(to_bits(x), g.cpu().numpy(), b.cpu().numpy(), 1e-5)
    assert np.array_equal(to_bits(y), want)


def test_layernorm_f32(dev):
    _case("layernorm f32")
    T, C = 3, 96
    x = _f16((T, C), 12, dev).float() * 20
    g, b = _w(C, 13, dev), _w(C, 14, dev, 0.0, 0.1)
    y = ops.layer_norm(x, g, b, 1e-5)
    want = np.empty((T, C), np.float32)
    O.lib().oracle_layernorm(O._ptr(x.cpu().numpy()), O._ptr(want), O._ptr(g.cpu().numpy()), O._ptr(b.cpu().numpy()),
                             T, C, 1e-5)
    np.testing.assert_allclose(y.cpu().numpy(), want, rtol=2e-7, atol=1e-7)


# ------------------------------------------------------------------ gated RMSNorm

@pytest.mark.parametrize("T,D,groups,zpad", [(16384, 3072, 1, 0), (64, 3072, 1, 640), (37, 1024, 4, 8), (5, 300, 3, 0),
                                               (256, 6144, 2, 0), (300, 2048, 1, 24), (40, 8192, 1, 0),
                                               (24, 9216, 1, 0)])
def test_gated_rmsnorm_f16(dev, T, D, groups, zpad):
    _case(f"gated rmsnorm T={T} D={D} groups={groups} zpad={zpad}")
    y = _f16((T, D), 15, dev)
    zfull = _f16((T, D + zpad), 16, dev)
    z = zfull[:, :D]
    w = _w(D, 17, dev)
    out = ops.gated_rms_norm(y, z, w, groups, 1e-5)
    want = O.gated_rmsnorm_f16(to_bits(y), to_bits(z), w.cpu().numpy(), groups, 1e-5)
    assert_f16_close(to_bits(out), want, what=f"gated {T}x{D}/{groups}")


def test_gated_rmsnorm_inplace(dev):
    _case("gated rmsnorm in place")
    y = _f16((100, 3072), 18, dev)
    z = _f16((100, 3072), 19, dev)
    w = _w(3072, 20, dev)
    want = O.gated_rmsnorm_f16(to_bits(y), to_bits(z), w.cpu().numpy(), 1, 1e-5)
    ops.gated_rms_norm(y, z, w, 1, 1e-5, out=y)
    assert_f16_close(to_bits(y), want, what="gated in place")


@pytest.mark.parametrize("D", [1024, 3072])
def test_gated_rmsnorm_every_gate(dev, D):
    """Every f16 gate value, one per element (subnormals, +-65504, +-inf and NaNs, in bit-pattern
    order), under random y: within 2 ulp of the oracle, NaN exactly where the oracle has NaN. D = 1024
    runs the one-wave kernel, D = 3072 (the Granite width) three waves per row; the last of its 22 rows
    is padded with zero gates."""
    _case(f"gated rmsnorm every gate value D={D}")
    rows = -(-65536 // D)
    codes = np.zeros(rows * D, dtype=np.uint16)
    codes[:65536] = np.arange(65536, dtype=np.uint16)
    z = torch.from_numpy(codes.view(np.float16).reshape(rows, D).copy()).to(dev)
    y = _f16((rows, D), 57, dev)
    w = _w(D, 58, dev)
    out = ops.gated_rms_norm(y, z, w, 1, 1e-5)
    want = O.gated_rmsnorm_f16(to_bits(y), to_bits(z), w.cpu().numpy(), 1, 1e-5)
    assert_f16_close(to_bits(out), want, what="gated every gate")


@pytest.mark.parametrize("groups", [1, 2])
def test_gated_rmsnorm_f32(dev, groups):
    """f32 I/O (the reference's activation type) at the Granite width, against the oracle's f32 op."""
    T, D = 64, 3072
    _case(f"gated rmsnorm f32 groups={groups}")
    y = _f16((T, D), 59, dev).float()
    z = (_f16((T, D), 60, dev) * 4).float()
    w = _w(D, 61, dev)
    out = ops.gated_rms_norm(y, z, w, groups, 1e-5)
    want = y.cpu().numpy().copy()
    O.lib().oracle_gated_rmsnorm(O._ptr(want), O._ptr(z.cpu().numpy()), D, O._ptr(w.cpu().numpy()), T, D, groups, 1e-5)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-30)


# ------------------------------------------------------------------ q/k norm + RoPE

def _qk_case(dev, T, n_q, n_kv, hd, n_pos, positions, norm, theta=1e6, stream=21, dtype=torch.float16):
    stride = (n_q + 2 * n_kv) * hd
    qkv = _f16((T, stride), stream, dev)
    if dtype == torch.float32:
        qkv = qkv.float()
    wqk = _w(2 * hd, stream + 1, dev) if norm else None
    cs = ops.rope_table(theta, hd, n_pos)
    before = qkv.cpu().numpy().copy()
    pos_t = None if positions is None else torch.from_numpy(positions).to(dev)
    ops.qk_norm_rope(qkv, n_q, n_kv, hd, torch.from_numpy(cs).to(dev), 1e-6, wqk=wqk, positions=pos_t)
    w_np = None if wqk is None else wqk.cpu().numpy()
    if dtype == torch.float16:
        want = O.qk_norm_rope_f16(before.view(np.uint16), n_q, n_kv, hd, cs, n_pos, 1e-6, wqk=w_np, positions=positions)
        got = to_bits(qkv)
        assert_f16_close(got, want, what=f"qk rope T={T} heads={n_q}+{n_kv} hd={hd}")
        # V heads are neither read nor written.
        v0 = (n_q + n_kv) * hd
        assert np.array_equal(got[:, v0:], before.view(np.uint16)[:, v0:])
    else:
        want = O.qk_norm_rope_f32(before, n_q, n_kv, hd, cs, n_pos, 1e-6, wqk=w_np, positions=positions)
        np.testing.assert_allclose(qkv.cpu().numpy(), want, rtol=1e-6, atol=1e-6)


def test_qk_rope_decode(dev):
    _case("qk rope Qwen3-0.6B decode, random positions")
    cfg = wl.QWEN3_DECODE
    pos = wl.uniform_ids(cfg.T, cfg.n_pos, 7)
    _qk_case(dev, cfg.T, cfg.n_q, cfg.n_kv, cfg.hd, cfg.n_pos, pos, True)


def test_qk_rope_prefill(dev):
    _case("qk rope Qwen3-4B prefill")
    cfg = wl.QWEN3_PREFILL
    pos = (np.arange(cfg.T) % cfg.seq).astype(np.int32)
    _qk_case(dev, cfg.T, cfg.n_q, cfg.n_kv, cfg.hd, cfg.seq, pos, True)


@pytest.mark.parametrize("n_q,n_kv,hd,norm,dtype", [
    (16, 8, 128, False, torch.float16),  # rotation only (rope.comp flags 0)
    (2, 1, 64, True, torch.float16),
    (3, 1, 96, True, torch.float16),     # hd/2 not a power-of-two lane count: fallback kernel
    (4, 2, 256, True, torch.float16),
    (2, 1, 64, True, torch.float32),
    (8, 2, 128, True, torch.float32),
    (32, 8, 128, True, torch.float32),   # Qwen3-4B heads in f32: ten passes, two rolling items of five
    (64, 16, 128, True, torch.float16),  # ten passes in f16
    (64, 8, 128, True, torch.float16),   # nine passes: the batch kernel
])
def test_qk_rope_shapes(dev, n_q, n_kv, hd, norm, dtype):
    _case(f"qk rope n_q={n_q} n_kv={n_kv} hd={hd} norm={norm} {dtype}")
    pos = wl.uniform_ids(37, 512, 22)
    _qk_case(dev, 37, n_q, n_kv, hd, 512, pos, norm, theta=1e4, dtype=dtype)


def test_qk_rope_rows_beyond_one_launch(dev):
    """More rows than the persistent grid takes in one launch (at most 64 per wave: with the 8192
    resident waves a one-pass head layout allows, 524288 rows), so the op runs in several launches;
    some positions fall outside the table."""
    _case("qk rope 600000 rows (several launches)")
    T, n_q, n_kv, hd, n_pos = 600000, 1, 1, 64, 4096
    rng = np.random.default_rng(27)
    pos = rng.integers(0, n_pos, T).astype(np.int32)
    pos[rng.integers(0, T, 50)] = -5
    pos[rng.integers(0, T, 50)] = n_pos
    _qk_case(dev, T, n_q, n_kv, hd, n_pos, pos, True)


def test_qk_rope_pos0_and_out_of_range(dev):
    _case("qk rope pos0 form and out-of-range positions")
    # pos0 + row (the reference's GPU ABI)
    T, n_q, n_kv, hd = 6, 4, 2, 128
    stride = (n_q + 2 * n_kv) * hd
    qkv = _f16((T, stride), 23, dev)
    cs = ops.rope_table(1e6, hd, 16)
    before = to_bits(qkv).copy()
    ops.qk_norm_rope(qkv, n_q, n_kv, hd, torch.from_numpy(cs).to(dev), 1e-6, pos0=3)
    want = O.qk_norm_rope_f16(before, n_q, n_kv, hd, cs, 16, 1e-6, pos0=3)
    assert_f16_close(to_bits(qkv), want, what="qk rope pos0")
    # rows whose position falls outside the table stay untouched
    qkv = _f16((T, stride), 24, dev)
    before = to_bits(qkv).copy()
    pos = np.array([0, -1, 15, 16, 1 << 30, 2], np.int32)
    ops.qk_norm_rope(qkv, n_q, n_kv, hd, torch.from_numpy(cs).to(dev), 1e-6, positions=torch.from_numpy(pos).to(dev))
    got = to_bits(qkv)
    for r in (1, 3, 4):
        assert np.array_equal(got[r], before[r])
    want = O.qk_norm_rope_f16(before, n_q, n_kv, hd, cs, 16, 1e-6, positions=pos)
    assert_f16_close(got, want, what="qk rope out of range")


def test_qk_rope_position_zero_is_norm_only(dev):
    _case("qk rope position 0 = identity rotation")
    T, n_q, n_kv, hd = 4, 2, 1, 128
    qkv = _f16((T, (n_q + 2 * n_kv) * hd), 25, dev)
    wqk = _w(2 * hd, 26, dev)
    x = qkv.clone()
    cs = torch.from_numpy(ops.rope_table(1e6, hd, 8)).to(dev)
    ops.qk_norm_rope(qkv, n_q, n_kv, hd, cs, 1e-6, wqk=wqk, positions=torch.zeros(T, dtype=torch.int32, device=dev))
    heads = x[:, :(n_q + n_kv) * hd].reshape(T * (n_q + n_kv), hd)
    wq = torch.cat([wqk[:hd].repeat(n_q, 1), wqk[hd:].repeat(n_kv, 1)]).repeat(T, 1)
    normed = torch.empty_like(heads)
    for i in range(heads.shape[0]):
        normed[i] = ops.rms_norm(heads[i:i + 1], wq[i].contiguous(), 1e-6)[0]
    got = to_bits(qkv[:, :(n_q + n_kv) * hd]).reshape(-1, hd)
    assert np.array_equal(got, to_bits(normed))


# ------------------------------------------------------------------ KV-cache store, fused and alone

def _caches(rows, width, dev):
    """float16 caches pre-filled with 0xFFFF (a NaN pattern) so rows the op must not write show up."""
    kc = torch.full((rows, width), -1, dtype=torch.int16, device=dev).view(torch.float16)
    return kc, kc.clone()


def _kv_case(dev, T, n_q, n_kv, hd, n_pos, positions, dtype=torch.float16, stream=61, pos0=0):
    stride = (n_q + 2 * n_kv) * hd
    qkv = _f16((T, stride), stream, dev)
    if dtype == torch.float32:
        qkv = qkv.float()
    wqk = _w(2 * hd, stream + 1, dev)
    cs = ops.rope_table(1e6, hd, n_pos)
    before = qkv.cpu().numpy().copy()
    kc, vc = _caches(n_pos, n_kv * hd, dev)
    pos_t = None if positions is None else torch.from_numpy(positions).to(dev)
    ops.qk_norm_rope_kv(qkv, n_q, n_kv, hd, torch.from_numpy(cs).to(dev), 1e-6, kc, vc, wqk=wqk, positions=pos_t,
                        pos0=pos0)
    src = before.view(np.uint16) if dtype == torch.float16 else before
    want, wk, wv = O.qk_norm_rope_kv(src, n_q, n_kv, hd, cs, n_pos, 1e-6, wqk=wqk.cpu().numpy(), positions=positions,
                                     pos0=pos0)
    gk, gv = to_bits(kc), to_bits(vc)
    what = f"qk rope+kv T={T} heads={n_q}+{n_kv} hd={hd} {dtype}"
    if dtype == torch.float16:
        got = to_bits(qkv)
        assert_f16_close(got, want, what=what)
        # the k cache holds exactly the rotated k heads the op wrote back; v is copied bit for bit
        kw = n_kv * hd
        rows_k = got[:, n_q * hd:n_q * hd + kw]
        p = positions if positions is not None else pos0 + np.arange(T)
        ok = (p >= 0) & (p < n_pos)
        assert np.array_equal(gk[p[ok]], rows_k[ok])
        assert_f16_close(gk, wk, what=what + " k cache")
        assert np.array_equal(gv, wv)
        assert np.array_equal(got[:, (n_q + n_kv) * hd:], before.view(np.uint16)[:, (n_q + n_kv) * hd:])  # v untouched
    else:
        np.testing.assert_allclose(qkv.cpu().numpy(), want, rtol=1e-6, atol=1e-6)
        assert_f16_close(gk, wk, what=what + " k cache")
        assert np.array_equal(gv, wv)
    untouched = ~(wk != 0xFFFF).any(axis=1)
    assert (gk[untouched] == 0xFFFF).all() and (gv[untouched] == 0xFFFF).all()


def test_qk_rope_kv_prefill(dev):
    """Qwen3-4B prefill of one 8192-token sequence: every position's k and v land in the caches."""
    _case("qk rope + kv store, Qwen3-4B 8192-token prefill")
    cfg = wl.QWEN3_PREFILL
    _kv_case(dev, cfg.T, cfg.n_q, cfg.n_kv, cfg.hd, cfg.T, np.arange(cfg.T, dtype=np.int32))


@pytest.mark.parametrize("n_q,n_kv,hd,dtype", [
    (16, 8, 128, torch.float16),   # Qwen3-0.6B decode
    (2, 1, 64, torch.float16),
    (3, 1, 96, torch.float16),     # no fused kernel for this head size: rope then store
    (64, 8, 128, torch.float16),   # 80 heads: ten passes, two items of five
    (64, 12, 128, torch.float16),  # 88 heads: eleven passes, no fused kernel: rope then store
    (32, 8, 128, torch.float32),   # f32, 4 heads per pass: 12 passes, two items of six
    (8, 2, 128, torch.float32),
    (32, 8, 128, torch.float16),   # Qwen3-4B heads: 6 passes, each token two work items of 3
    (40, 12, 128, torch.float16),  # 8 passes: two items of 4
    (16, 8, 128, torch.float32),   # f32, 4 heads per pass: 8 passes, two items of 4
])
def test_qk_rope_kv_shapes(dev, n_q, n_kv, hd, dtype):
    _case(f"qk rope + kv n_q={n_q} n_kv={n_kv} hd={hd} {dtype}")
    rng = np.random.default_rng(62)
    pos = rng.permutation(512)[:37].astype(np.int32)
    pos[[3, 9]] = [-1, 512]  # outside the table: untouched, no store
    _kv_case(dev, 37, n_q, n_kv, hd, 512, pos, dtype=dtype)


@pytest.mark.parametrize("n_q,n_kv", [(4, 2), (32, 8)])
def test_qk_rope_kv_pos0(dev, n_q, n_kv):
    _case(f"qk rope + kv store, pos0 form, heads {n_q}+{n_kv}")
    _kv_case(dev, 13, n_q, n_kv, 128, 16, None, pos0=5)  # rows 11 and 12 fall outside the 16-row table


def test_qk_rope_kv_rows_beyond_one_launch(dev):
    """The fused KV store over two work items per token (64 + 16 + 16 heads x 64: six passes) on more
    rows than one launch takes (at most 64 items per wave: 163,840 rows at the 1280 workgroups that
    stay resident), so the op runs in two launches; distinct positions, some outside the table."""
    _case("qk rope + kv store, 166000 rows (two launches)")
    T, n_q, n_kv, hd = 166000, 64, 16, 64
    rng = np.random.default_rng(63)
    pos = rng.permutation(T).astype(np.int32)
    pos[rng.integers(0, T, 40)] = -3
    _kv_case(dev, T, n_q, n_kv, hd, T, pos, stream=64)


@pytest.mark.parametrize("dtype,width,k_off,v_off", [
    (torch.float16, 1024, 4096, 5120),   # Qwen3-4B k/v columns
    (torch.float32, 1024, 4096, 5120),
    (torch.float16, 100, 7, 301),        # unaligned / odd width: per-element kernel
    (torch.float32, 24, 40, 8),
])
def test_store_kv(dev, dtype, width, k_off, v_off):
    """cpu::storeKv: f16 activations copied bit for bit, f32 rounded to f16; positions outside the
    cache skipped."""
    _case(f"store kv {dtype} width={width}")
    T, cols, cache_rows = 50, 6144, 40
    qkv = _f16((T, cols), 63, dev, std=300.0)
    if dtype == torch.float32:
        qkv = (qkv.float() * 3.3).contiguous()
        qkv[1, k_off] = 1e-7
        qkv[2, v_off] = 1e6
    rng = np.random.default_rng(64)
    pos = rng.integers(-3, cache_rows + 3, T).astype(np.int32)
    pos[:cache_rows] = rng.permutation(cache_rows)[:cache_rows]  # unique rows, then some out of range
    pos[cache_rows:] = np.array([-1, -2, cache_rows, cache_rows + 5, -7, cache_rows, 41, -1, 99, -3])[:T - cache_rows]
    kc, vc = _caches(cache_rows, width, dev)
    ops.store_kv(qkv, k_off, v_off, width, kc, vc, positions=torch.from_numpy(pos).to(dev))
    src = to_bits(qkv) if dtype == torch.float16 else qkv.cpu().numpy()
    wk, wv = O.store_kv(src, k_off, v_off, width, cache_rows, positions=pos)
    assert np.array_equal(to_bits(kc), wk) and np.array_equal(to_bits(vc), wv)
    kc, vc = _caches(cache_rows, width, dev)
    ops.store_kv(qkv, k_off, v_off, width, kc, vc, pos0=30)  # rows 10.. of the batch fall past the cache
    wk, wv = O.store_kv(src, k_off, v_off, width, cache_rows, pos0=30)
    assert np.array_equal(to_bits(kc), wk) and np.array_equal(to_bits(vc), wv)


# ------------------------------------------------------------------ residual add + RMSNorm

@pytest.mark.parametrize("T,C,dtype", [
    (8192, 2560, torch.float16),   # Qwen3-4B prefill (one round, two rows per wave)
    (64, 1024, torch.float16),     # one round, one row per wave
    (8191, 2000, torch.float16),   # one round, two rows per wave, the last wave one short; lanes past the row end
    (12288, 2560, torch.float16),  # three rows of five chunks: more than the one-round budget, persistent waves
    (7, 100, torch.float16),       # odd width: generic kernel
    (3, 20000, torch.float16),     # four waves per row
    (33, 1536, torch.float32),
    (8192, 1024, torch.float32),   # f32, one round, two rows per wave
])
def test_add_rmsnorm(dev, T, C, dtype):
    _case(f"add + rmsnorm {T}x{C} {dtype}")
    x = _f16((T, C), 65, dev, std=4.0)
    d = _f16((T, C), 66, dev, std=0.5)
    if dtype == torch.float32:
        x, d = x.float(), d.float()
    d[1] = -x[1]  # a row that cancels to zero: the eps-only scale
    w = _w(C, 67, dev)
    x0, d0 = x.cpu().numpy().copy(), d.cpu().numpy()
    xn = ops.add_rms_norm(x, d, w, 1e-6)
    if dtype == torch.float16:
        wx, wn = O.add_rmsnorm_f16(x0.view(np.uint16), d0.view(np.uint16), w.cpu().numpy(), 1e-6)
        assert np.array_equal(to_bits(x), wx)  # the residual sum is exact f32 then one RNE: bit-exact
        assert_f16_close(to_bits(xn), wn, what=f"add+rmsnorm {T}x{C}")
    else:
        want_n = np.empty_like(x0)
        O.lib().oracle_add_rmsnorm(O._ptr(x0), O._ptr(np.ascontiguousarray(d0)), O._ptr(want_n),
                                   O._ptr(w.cpu().numpy()), T, C, 1e-6)
        assert np.array_equal(x.cpu().numpy().view(np.uint32), x0.view(np.uint32))
        np.testing.assert_allclose(xn.cpu().numpy(), want_n, rtol=2e-7, atol=0)


def test_add_rmsnorm_rejects_aliasing(dev):
    x = _f16((4, 256), 68, dev)
    with pytest.raises(NekoError):
        ops.add_rms_norm(x, x.clone(), _w(256, 69, dev), 1e-6, out=x)
    buf = _f16((5, 256), 75, dev)
    with pytest.raises(NekoError):  # xn one row past x: the rows overlap
        ops.add_rms_norm(buf[:4], x.clone(), _w(256, 69, dev), 1e-6, out=buf[1:])


def test_partial_overlaps_rejected(dev):
    """Outputs are the input rows themselves (same address and stride) or disjoint from them: the
    persistent waves load later rows while storing earlier ones, so any other overlap would race.
    Each rejected call leaves its buffers untouched; the exact in-place forms still run."""
    _case("partial overlaps rejected")
    buf = _f16((9, 512), 70, dev)
    before = to_bits(buf).copy()
    w = _w(256, 71, dev)
    x = buf[:8, :256]
    z = _f16((8, 256), 72, dev)
    bad = [
        lambda: ops.rms_norm(x, w, 1e-6, out=buf[1:9, :256]),  # one row down
        lambda: ops.rms_norm(x, w, 1e-6, out=buf[:8, 8:264]),  # eight columns right
        lambda: ops.layer_norm(x, w, w, 1e-5, out=buf[1:9, :256]),
        lambda: ops.gated_rms_norm(x, z, w, 1, 1e-5, out=buf[1:9, :256]),
        lambda: ops.gated_rms_norm(x, z, w, 1, 1e-5, out=z),  # out over the gate operand
        lambda: ops.silu_mul(buf[:8], out=buf[:8, 256:]),  # out over the up halves
        lambda: ops.gelu(buf.view(-1)[:4000], out=buf.view(-1)[8:4008]),
    ]
    for i, call in enumerate(bad):
        with pytest.raises(NekoError):
            call()
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(buf), before)
    want = O.swiglu_f16(to_bits(buf[:8]))
    ops.silu_mul(buf[:8], out=buf[:8, :256])  # over the gate halves: each chunk rewritten by its reader
    assert_f16_close(to_bits(buf[:8, :256]), want, what="swiglu over its gate halves")


# ------------------------------------------------------------------ SwiGLU / GELU

@pytest.mark.parametrize("T,I", [(64, 3072), (8192, 9728), (16384, 4096), (2, 100), (3, 7)])
def test_swiglu_f16(dev, T, I):
    _case(f"swiglu T={T} I={I}")
    h = _f16((T, 2 * I), 27, dev)
    got = ops.silu_mul(h)
    want = O.swiglu_f16(to_bits(h))
    d = assert_f16_close(to_bits(got), want, what=f"swiglu {T}x{I}")
    assert np.count_nonzero(d > 1) == 0


def test_swiglu_all_gates(dev):
    _case("swiglu every fp16 gate value")
    gates = np.arange(65536, dtype=np.uint16)
    ups = np.array([0x3C00, 0xBC00, 0x3555, 0x7BFF, 0x0001, 0x4900], np.uint16)  # 1, -1, 1/3, max, min sub, 10
    h = np.empty((len(ups), 2 * 65536), np.uint16)
    h[:, :65536] = gates
    h[:, 65536:] = ups[:, None]
    ht = torch.from_numpy(h.view(np.float16)).to(dev)
    got = to_bits(ops.silu_mul(ht))
    want = O.swiglu_f16(h)
    assert_f16_close(got, want, max_ulp=1, what="swiglu all gates")


def test_swiglu_strided_f32(dev):
    _case("swiglu strided and f32")
    T, I = 9, 1000
    buf = _f16((T, 2 * I + 16), 28, dev)
    h = buf[:, :2 * I]
    out = torch.zeros((T, I + 8), dtype=torch.float16, device=dev)
    ops.silu_mul(h, out=out[:, :I])
    assert_f16_close(to_bits(out[:, :I]), O.swiglu_f16(to_bits(h)), what="swiglu strided")
    assert torch.count_nonzero(out[:, I:]) == 0
    hf = h.float() * 6
    want = np.empty((T, I), np.float32)
    O.lib().oracle_silu_mul(O._ptr(hf.cpu().numpy()), O._ptr(want), T, I)
    np.testing.assert_allclose(ops.silu_mul(hf).cpu().numpy(), want, rtol=4e-7, atol=1e-30)


def test_gelu_all_halves(dev):
    _case("gelu every fp16 value")
    x = np.arange(65536, dtype=np.uint16)
    got = to_bits(ops.gelu(torch.from_numpy(x.view(np.float16)).to(dev)))
    assert_f16_close(got, O.gelu_f16(x), what="gelu all halves")


@pytest.mark.parametrize("n", [128 * 3072, 1, 7, 4099])
def test_gelu_sizes(dev, n):
    _case(f"gelu n={n}")
    x = _f16((n,), 29, dev)
    assert_f16_close(to_bits(ops.gelu(x)), O.gelu_f16(to_bits(x)), what=f"gelu n={n}")


def test_gelu_f32_inplace(dev):
    _case("gelu f32 in place")
    x = _f16((1000,), 30, dev).float() * 4
    want = np.array([O.lib().oracle_gelu(float(v)) for v in x.cpu().numpy()], np.float32)
    ops.gelu(x, out=x)
    np.testing.assert_allclose(x.cpu().numpy(), want, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------ embedding gather

def _table(fmt, rows, C, stream):
    x = wl.normal_f16((rows, C), 0.0, 0.02, stream, "cpu").float().numpy()
    table, used = ops.quantize_rows(fmt, x)
    assert used == fmt
    return table


@pytest.mark.parametrize("fmt", [ops.FMT_F16, ops.FMT_FP8, ops.FMT_FP4])
def test_embed_quant_gather_full(dev, fmt):
    """Qwen3-1.7B-shaped tied table, 16384 Zipf ids: bit-exact."""
    cfg = wl.QUANT_GATHER
    _case(f"embed gather fmt={fmt} {cfg.vocab}x{cfg.C}")
    x = wl.normal_f16((cfg.vocab, cfg.C), 0.0, 0.02, 31, dev).float().cpu().numpy()
    table, _ = ops.quantize_rows(fmt, x)
    ids = wl.zipf_ids(cfg.T, cfg.vocab, cfg.s, 32)
    got = ops.embed(torch.from_numpy(ids).to(dev), torch.from_numpy(table).to(dev), fmt, cfg.C)
    want = O.embed(ids, table, fmt, cfg.C)
    assert np.array_equal(to_bits(got), want)


@pytest.mark.parametrize("fmt", [ops.FMT_FP8, ops.FMT_FP4])
def test_embed_every_code_and_scale(dev, fmt):
    """Every code under scales spanning f16 subnormals to the maximum, both signs: bit-exact, f16 and f32 out."""
    _case(f"embed every code fmt={fmt}")
    C = 256
    scales = np.array([0x0001, 0x0003, 0x03FF, 0x0400, 0x1400, 0x2E66, 0x3C00, 0x4400, 0x5BFF, 0x7800, 0x7BFF,
                       0x8001, 0xBC00, 0xFBFF, 0x0000, 0x8000], np.uint16)
    rb = ops.quant_row_bytes(fmt, C)
    table = np.zeros((len(scales), rb), np.uint8)
    for r, s in enumerate(scales):
        if fmt == ops.FMT_FP8:
            table[r, :C] = np.arange(256, dtype=np.uint8)
            table[r, C:C + 16].view(np.uint16)[:] = s
        else:
            nib = np.arange(C, dtype=np.uint8) % 16
            blocks = nib.reshape(C // 32, 32)
            packed = (blocks[:, :16] | (blocks[:, 16:] << 4)).astype(np.uint8)
            table[r, :C // 2] = packed.reshape(-1)
            table[r, C // 2:C // 2 + 16].view(np.uint16)[:] = s
    ids = np.arange(len(scales), dtype=np.int32)[::-1].copy()
    tt = torch.from_numpy(table).to(dev)
    it = torch.from_numpy(ids).to(dev)
    got16 = ops.embed(it, tt, fmt, C)
    assert np.array_equal(to_bits(got16), O.embed(ids, table, fmt, C))
    got32 = ops.embed(it, tt, fmt, C, out_dtype=torch.float32)
    want32 = O.embed(ids, table, fmt, C, out_f16=False)
    assert np.array_equal(got32.cpu().numpy().view(np.uint32), want32.view(np.uint32))


@pytest.mark.parametrize("fmt", [ops.FMT_F16, ops.FMT_FP8, ops.FMT_FP4])
def test_embed_scaled_granite(dev, fmt):
    """Granite's gather (granite_model.cpp:298-301): every dequantised value times the model's
    embedding_multiplier in f32 -- one IEEE f32 multiply of the exact value -- and f16 output one RNE
    rounding of that. Pinned by the closed form: the oracle's exact f32 gather times the multiplier in
    numpy float32, then numpy's RNE to f16. Multipliers: Granite-4.0's 12, 0.3 (rounds), 2^-20
    (exact), 70000 (f16 overflow to inf), on every code of every format and 3000 random tokens over
    Granite's 1536-wide rows."""
    _case(f"embed scaled fmt={fmt}")
    C, V = 1536, 1000
    x = wl.normal_f16((V, C), 0.0, 0.02, 36, "cpu").float().numpy()
    x[0, :256] = np.linspace(-6.0, 6.0, 256, dtype=np.float32) * 0.02  # every magnitude class in one row
    table, used = ops.quantize_rows(fmt, x)
    assert used == fmt
    ids = np.concatenate([np.zeros(4, np.int32), wl.uniform_ids(2996, V, 37)])
    tt, it = torch.from_numpy(table).to(dev), torch.from_numpy(ids).to(dev)
    base = O.embed(ids, table, fmt, C, out_f16=False)
    for mult in (12.0, 0.3, 2.0 ** -20, 70000.0):
        want32 = base * np.float32(mult)
        got32 = ops.embed(it, tt, fmt, C, out_dtype=torch.float32, scale=mult).cpu().numpy()
        assert np.array_equal(got32.view(np.uint32), want32.view(np.uint32)), f"f32 out, multiplier {mult}"
        got16 = ops.embed(it, tt, fmt, C, scale=mult)
        assert np.array_equal(to_bits(got16), want32.astype(np.float16).view(np.uint16)), f"f16 out, multiplier {mult}"


@pytest.mark.parametrize("fmt", [ops.FMT_FP8, ops.FMT_FP4])
@pytest.mark.parametrize("C", [96, 2080, 4096, 5152])
def test_embed_widths(dev, fmt, C):
    """Row widths around the kernel's steps of 256 output chunks, whose block scales one load per lane
    brings in: a few blocks (96), one step and a few chunks more with an odd block count (2080: 65
    blocks), two whole steps (4096), and an odd count past two steps (5152: 161 blocks). The table's last
    row is among the ids (its scale area ends the buffer). Bit-exact, f16 and f32 out."""
    _case(f"embed widths fmt={fmt} C={C}")
    V, T = 40, 130
    table = _table(fmt, V, C, 41)
    ids = wl.uniform_ids(T, V, 42)
    ids[:2] = [V - 1, 0]
    tt, it = torch.from_numpy(table).to(dev), torch.from_numpy(ids).to(dev)
    assert np.array_equal(to_bits(ops.embed(it, tt, fmt, C)), O.embed(ids, table, fmt, C))
    got32 = ops.embed(it, tt, fmt, C, out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), O.embed(ids, table, fmt, C, out_f16=False).view(np.uint32))


def test_embed_gpt2_wpe(dev):
    """GPT-2 wte + wpe (f32 add, then one f16 rounding) at the configured shape: bit-exact."""
    cfg = wl.GPT2_CHAIN
    _case("embed gpt2 wte+wpe")
    wte = wl.normal_f16((cfg.vocab, cfg.C), 0.0, 0.02, 33, "cpu").numpy()
    wpe = wl.normal_f16((cfg.n_ctx, cfg.C), 0.0, 0.02, 34, "cpu").numpy()
    ids = wl.uniform_ids(cfg.T, cfg.vocab, 35)
    table = wte.view(np.uint8).reshape(cfg.vocab, 2 * cfg.C)
    for pos0 in (0, cfg.n_ctx - cfg.T):
        got = ops.embed(torch.from_numpy(ids).to(dev), torch.from_numpy(table).to(dev), ops.FMT_F16, cfg.C,
                        wpe=torch.from_numpy(wpe).to(dev), pos0=pos0)
        want = O.embed(ids, table, ops.FMT_F16, cfg.C, wpe=wpe.view(np.uint16), pos0=pos0)
        assert np.array_equal(to_bits(got), want)
    with pytest.raises(NekoError):
        ops.embed(torch.from_numpy(ids).to(dev), torch.from_numpy(table).to(dev), ops.FMT_F16, cfg.C,
                  wpe=torch.from_numpy(wpe).to(dev), pos0=cfg.n_ctx - cfg.T + 1)


@pytest.mark.parametrize("fmt", [ops.FMT_F16, ops.FMT_FP8, ops.FMT_FP4])
def test_embed_chunked_table_and_wpe(dev, fmt):
    """A table split into row chunks gathered with one call per chunk; quantized rows + wpe; f32 out."""
    _case(f"embed chunked fmt={fmt}")
    V, C, T = 1000, 512, 300
    table = _table(fmt, V, C, 36)
    ids = wl.uniform_ids(T, V, 37)
    ids[:3] = [0, V - 1, 417]
    wpe = wl.normal_f16((T + 5, C), 0.0, 0.02, 38, "cpu").numpy()
    out = torch.zeros((T, C), dtype=torch.float32, device=dev)
    it = torch.from_numpy(ids).to(dev)
    for r0, r1 in ((0, 417), (417, 1000)):
        chunk = torch.from_numpy(table[r0:r1].copy()).to(dev)
        ops.embed(it, chunk, fmt, C, row_base=r0, wpe=torch.from_numpy(wpe).to(dev), pos0=5, out=out)
    want = O.embed(ids, table, fmt, C, wpe=wpe.view(np.uint16), pos0=5, out_f16=False)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_embed_fallback_layouts(dev):
    """Odd widths and unaligned rows take the per-element kernel: still bit-exact."""
    _case("embed fallback layouts")
    V, C, T = 50, 100, 40
    tab = wl.normal_f16((V, C), 0.0, 0.02, 39, "cpu").numpy().view(np.uint8).reshape(V, 2 * C)
    ids = wl.uniform_ids(T, V + 10, 40)  # some ids outside the table: rows left as they were
    out = torch.full((T, C), 7.0, dtype=torch.float16, device=dev)
    ops.embed(torch.from_numpy(ids).to(dev), torch.from_numpy(tab).to(dev), ops.FMT_F16, C, out=out)
    want = np.full((T, C), 0x4700, np.uint16)
    want = O.embed(ids, tab, ops.FMT_F16, C, out=want)
    assert np.array_equal(to_bits(out), want)


def test_embed_empty_and_invalid(dev):
    _case("embed empty and invalid")
    tab = torch.zeros((4, 64), dtype=torch.uint8, device=dev)
    none = torch.zeros(0, dtype=torch.int32, device=dev)
    assert ops.embed(none, tab, ops.FMT_F16, 32).shape == (0, 32)
    with pytest.raises(NekoError):
        ops.embed(torch.zeros(2, dtype=torch.int32, device=dev), tab, ops.FMT_FP8, 48)  # C % 32 != 0


# ------------------------------------------------------------------ load-time quantiser

def _quant_source(rows, cols, seed):
    """~N(0, 0.02) weights with blocks that reach every branch of the encoders: all-zero rows and
    blocks, outliers, tiny blocks whose scales are f16 subnormals or round to zero, a block whose
    FP8/FP4 scale overflows f16, exact code values, and sign mixes."""
    rng = np.random.default_rng(seed)
    x = (0.02 * rng.standard_normal((rows, cols))).astype(np.float32)
    x[0] = 0.0
    x[1, 32:64] = 0.0
    x[2, 5] = 1.5
    x[2, 40] = -3e-6
    x[3, :64] *= 1e-5                 # scales near and below the smallest f16 subnormals
    x[3, 64:96] = 1e-12               # rounds to a zero scale
    x[4, :32] *= 1e9                  # FP8 and FP4 scales overflow to inf (codes 0)
    x[5, :32] = np.tile(np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float32), 4) * np.float32(0.125)
    x[5, 32:64] = -x[5, :32]
    x[6] = rng.standard_normal(cols).astype(np.float32) * (10.0 ** rng.integers(-6, 3, cols)).astype(np.float32)
    return x


@pytest.mark.parametrize("fmt", [ops.FMT_F16, ops.FMT_FP8, ops.FMT_FP4])
@pytest.mark.parametrize("src_dtype", [torch.float32, torch.float16])
def test_quantize_gpu_bitexact(dev, fmt, src_dtype):
    """The device quantiser writes the same bytes as the oracle (itself pinned to the reference's
    quantizeMatrix) and as the host C-ABI encoder, codes, scales and padding."""
    _case(f"quantize fmt={fmt} src={src_dtype}")
    x = _quant_source(512, 2048, 81 + fmt)
    if src_dtype == torch.float16:
        x = np.clip(x, -60000, 60000).astype(np.float16).astype(np.float32)  # f16 sources: exact widening
    src = torch.from_numpy(x).to(dev).to(src_dtype)
    got, used = ops.quantize(src, fmt)
    assert used == fmt
    want = O.quantize_rows(fmt, x)
    g = got.cpu().numpy()
    bad = np.argwhere(g != want)
    if bad.size:
        r, c = (int(v) for v in bad[0])
        cols = x.shape[1]
        codes = cols if fmt == ops.FMT_FP8 else cols // 2 if fmt == ops.FMT_FP4 else 2 * cols
        per = 32 if fmt == ops.FMT_FP8 else 16
        part = "code" if c < codes else "scale" if c < codes + cols // 16 else "padding"
        blk = c // per if part == "code" else (c - codes) // 2
        xb = x[r, 32 * blk:32 * blk + 32] if fmt != ops.FMT_F16 else x[r, c // 2:c // 2 + 1]
        pytest.fail(f"{len(bad)} bytes differ; first at row {r} byte {c} ({part}, block {blk}): got {g[r, c]:#04x} "
                    f"want {want[r, c]:#04x}; block amax {np.abs(xb).max():.9g}, scale want "
                    f"{want[r, codes + 2 * blk:codes + 2 * blk + 2].view(np.uint16)} got "
                    f"{g[r, codes + 2 * blk:codes + 2 * blk + 2].view(np.uint16)}; values {xb[:8]}")
    if src_dtype == torch.float32:
        host, _ = ops.quantize_rows(fmt, x)
        assert np.array_equal(host, want)


def _quant_edges():
    """Blocks aimed at the encoders' rounding edges. FP4 fits: blocks whose amax is 6, so the first
    fit's scale is exactly 1 and it rounds the raw magnitudes -- every tie of the E2M1 ladder (0.25 ...
    5.0, 5.0 the one the reference rounds up where nearest-even rounds down) and its f32 neighbours,
    alone and repeated so that the refit's scale depends on them. FP8: blocks whose f16 scale is a
    subnormal rounded well below amax/448, so the scaled weights reach past 448 (the codes clamp to
    0x7E). FP4 codes: blocks whose final scale is 1 with exact ties in them (below)."""
    f = np.float32
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], f)
    near = np.concatenate([ties, np.nextafter(ties, f(0)), np.nextafter(ties, f(10))])
    rows = []
    rng = np.random.default_rng(17)
    for k in range(30):
        blk = np.resize(near[rng.permutation(near.size)], 32).astype(f)
        blk[k % 32] = 6.0
        if k % 3 == 1:
            blk[:24] = 5.0
            blk[24] = 6.0
        if k % 3 == 2:
            blk[1::2] *= -1
        rows.append(blk)
    for m in (1.1, 1.4, 1.49, 2.3, 2.6, 3.3, 5.5, 9.7, 17.3, 33.1):
        amax = f(448.0 * m * 2.0 ** -24)
        blk = (rng.uniform(-1, 1, 32) * amax).astype(f)
        blk[3] = amax
        blk[7] = -amax
        blk[11] = f(0.97) * amax
        rows.append(blk)
    # FP4 encoder ties: 0.75 / 1.75 / 3.5 (which nearest-even rounds up and the reference down), each
    # balanced by ties the fits round down (1.25, 2.5), among exact grid values and small magnitudes of
    # either sign (codes with no sign): the least-squares refit returns exactly 1, so the encoder sees
    # the ties exactly.
    for k in range(8):
        tie = np.array([0.75, 1.25, 1.75, 1.25, 1.25, 3.5, 2.5, 2.5], f) * rng.choice([-1, 1], 8).astype(f)
        small = np.array([-0.1, -0.25, 0.25, -0.0, 0.2, -0.24], f)
        grid = rng.choice(np.array([0.5, 1, 1.5, 2, 3, 4, 6, -0.5, -1, -2, -6], f), 17).astype(f)
        rows.append(np.concatenate([[f(6.0)], tie, small, grid]).astype(f)[rng.permutation(32)])
    return np.concatenate(rows).reshape(-1, 256)  # 48 blocks: 6 rows of 8


@pytest.mark.parametrize("fmt", [ops.FMT_FP8, ops.FMT_FP4])
def test_quantize_gpu_rounding_edges(dev, fmt):
    """The hardware E2M1 / E4M3 conversions, with their corrections, give the oracle's bytes at the
    encoders' rounding edges (the oracle is the reference's own arithmetic, pinned bit-exact to the
    compiled quantizeMatrix)."""
    _case(f"quantize rounding edges fmt={fmt}")
    x = _quant_edges()
    got, used = ops.quantize(torch.from_numpy(x).to(dev), fmt)
    assert used == fmt
    want = O.quantize_rows(fmt, x)
    assert np.array_equal(got.cpu().numpy(), want)
    # the edges are reached: FP4's first fits run at scale 1 (amax 6), FP8 scaled weights pass 448
    if fmt == ops.FMT_FP4:
        assert (np.abs(x.reshape(-1, 32)[:30]).max(axis=1) == 6.0).all()
        assert (want[:, 128:].view(np.uint16).reshape(-1)[40:] == 0x3C00).all()  # the tie blocks: scale 1
    else:
        s = want[:, 256:].view(np.float16).astype(np.float32)
        y = np.abs(x.reshape(-1, 8, 32)) / np.where(s > 0, s, np.inf)[:, :, None]
        assert (y.max(axis=2) > 452).sum() >= 5


def test_quantize_gpu_shapes(dev):
    _case("quantize: cols % 32 != 0 stores F16, strided source, then the gather reads the table back")
    x = _quant_source(40, 100, 91)
    got, used = ops.quantize(torch.from_numpy(x).to(dev), ops.FMT_FP4)
    assert used == ops.FMT_F16 and np.array_equal(got.cpu().numpy(), O.quantize_rows(ops.FMT_FP4, x))
    wide = torch.from_numpy(_quant_source(33, 512, 92)).to(dev)
    view = wide[:, :256]  # row stride 512, 256 columns
    for fmt in (ops.FMT_FP8, ops.FMT_FP4):
        got, _ = ops.quantize(view, fmt)
        want = O.quantize_rows(fmt, view.cpu().numpy())
        assert np.array_equal(got.cpu().numpy(), want)
        ids = np.arange(33, dtype=np.int32)[::-1].copy()
        out = ops.embed(torch.from_numpy(ids).to(dev), got, fmt, 256)
        assert np.array_equal(to_bits(out), O.embed(ids, want, fmt, 256))
    with pytest.raises(NekoError):
        ops.quantize(torch.zeros((4, 64), dtype=torch.float64, device=dev), ops.FMT_FP8)


def test_quantize_and_gather_full_table(dev):
    """Full size: the device quantiser encodes the 151936 x 2048 f32 table into the bytes whose sha256
    the reference's compiled quantizeMatrix gave (tests/golden/table_sha256.json), and the gather of
    16384 Zipf(1.1) ids from each encoded table equals the oracle's, bit for bit."""
    import hashlib
    import json
    import os

    import mm_tables as M

    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "table_sha256.json")) as f:
        want = json.load(f)
    x = M.qwen3_table_source(want["rows"], want["cols"])
    assert hashlib.sha256(x.data).hexdigest() == want["source_sha256"], "source table generator changed"
    C = want["cols"]
    src = torch.from_numpy(x).to(dev)
    del x
    cfg = wl.QUANT_GATHER
    ids = wl.zipf_ids(cfg.T, cfg.vocab, cfg.s, 32)
    idd = torch.from_numpy(ids).to(dev)
    for fmt, name in ((ops.FMT_F16, "f16"), (ops.FMT_FP8, "fp8"), (ops.FMT_FP4, "fp4")):
        _case(f"quantize + gather full table fmt={fmt}")
        tab, used = ops.quantize(src, fmt)
        assert used == fmt and tab.shape[1] == want[f"{name}_row_bytes"]
        host = tab.cpu().numpy()
        assert hashlib.sha256(host.data).hexdigest() == want[f"{name}_sha256"], name
        out = ops.embed(idd, tab, fmt, C)
        assert np.array_equal(to_bits(out), O.embed(ids, host, fmt, C))
        del tab, host, out


# ------------------------------------------------------------------ the GPT-2 op chain

def test_gpt2_chain(dev):
    """gather wte+wpe -> LayerNorm -> GELU, each stage against the oracle chain on the same data."""
    cfg = wl.GPT2_CHAIN
    _case("gpt2 chain")
    wte = wl.normal_f16((cfg.vocab, cfg.C), 0.0, 0.02, 41, "cpu").numpy()
    wpe = wl.normal_f16((cfg.n_ctx, cfg.C), 0.0, 0.02, 42, "cpu").numpy()
    ids = wl.uniform_ids(cfg.T, cfg.vocab, 43)
    g = _w(cfg.C, 44, dev, 1.0, 0.02)
    b = _w(cfg.C, 45, dev, 0.0, 0.02)
    table = wte.view(np.uint8).reshape(cfg.vocab, 2 * cfg.C)
    x = ops.embed(torch.from_numpy(ids).to(dev), torch.from_numpy(table).to(dev), ops.FMT_F16, cfg.C,
                  wpe=torch.from_numpy(wpe).to(dev))
    xw = O.embed(ids, table, ops.FMT_F16, cfg.C, wpe=wpe.view(np.uint16))
    assert np.array_equal(to_bits(x), xw)
    y = ops.layer_norm(x, g, b, cfg.eps)
    assert_f16_close(to_bits(y), O.layernorm_f16(xw, g.cpu().numpy(), b.cpu().numpy(), cfg.eps), what="chain LN")
    hf = _f16((cfg.T, cfg.F), 46, dev)
    assert_f16_close(to_bits(ops.gelu(hf)), O.gelu_f16(to_bits(hf)), what="chain GELU")
