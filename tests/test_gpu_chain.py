"""Layer-order chains on the GPU, each stage's output fed to the next and checked against the oracle.

Qwen3-4B prefill (qwen3_model.cpp:244-265) and a Granite-4.0-H Mamba layer (granite_model.cpp:278-287,
312-327) at their configured sizes. The weight matmuls between the ops run on the GPU
(neko_hip_matmul) with one-hot F16 weight rows -- row n holds a single 1.0 at column
(m n + a) mod K -- so each output is exactly one input value whatever the summation order: the chain
carries the GPU's own outputs forward through the real matmul kernels, and the oracle side of each
product is an exact column selection. The Qwen3 layer runs the real attention over each sequence's
caches (checked against the oracle at sampled tokens: within half an f16 ulp of its f32 result plus
2e-6 relative); the Mamba scan is outside this path, stood in for by a slice of the in_proj row.

Every op stage is compared with the oracle applied to the same input the GPU stage received (the
previous GPU stage's output): norms, RoPE and SwiGLU to the fp16 parity bar, residual sums, V heads,
the V cache and the selections bit for bit.
"""
import numpy as np
import pytest
import torch

from conftest import assert_f16_close, to_bits
from nekochat_amd import ops
from nekochat_amd import workloads as wl
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _onehot(n_out, n_in, mult, add, dev):
    """F16 weight rows (the reference's row layout: n_in halves) picking input column (mult n + add)
    mod n_in for output n; and those columns."""
    cols = (mult * np.arange(n_out, dtype=np.int64) + add) % n_in
    w = np.zeros((n_out, n_in), np.uint16)
    w[np.arange(n_out), cols] = 0x3C00
    return torch.from_numpy(w.view(np.uint8).reshape(n_out, 2 * n_in)).to(dev), cols


def _project(x, table, K, cols, what):
    """y = x W^T on the GPU (f16 out); checked equal to the selected columns of x."""
    y = ops.matmul(x, table, ops.FMT_F16, K, out_dtype=torch.float16)
    want = x[:, torch.from_numpy(cols).to(x.device)]
    assert torch.equal(y, want), f"{what}: one-hot product differs from the selected columns"
    return y


def test_qwen3_prefill_layer_chain(dev):
    """rmsNorm -> q/k/v projection -> per-head q/k norm + RoPE with the KV store -> attention -> o
    projection -> residual add + rmsNorm -> gate/up projection -> SwiGLU -> down projection
    accumulated into the residual; 4 sequences x 2048 tokens, hidden 2560."""
    cfg = wl.QWEN3_PREFILL
    T, C, H, KV, hd, F, S = cfg.T, cfg.C, cfg.n_q, cfg.n_kv, cfg.hd, cfg.I, cfg.seq
    QW, QH, KVW = cfg.qkv_stride, cfg.n_q * cfg.hd, cfg.n_kv * cfg.hd
    x = wl.normal_f16((T, C), 0.0, 1.0, 1, "cpu").to(dev)
    w_in = wl.weight_f32(C, 1.0, 0.05, 2, "cpu").to(dev)
    w_post = wl.weight_f32(C, 1.0, 0.05, 3, "cpu").to(dev)
    wqk = wl.weight_f32(2 * hd, 1.0, 0.05, 5, "cpu").to(dev)
    cs_host = ops.rope_table(cfg.theta, hd, S)
    cs = torch.from_numpy(cs_host).to(dev)

    _case("qwen3 chain: input rmsnorm")
    xn = ops.rms_norm(x, w_in, cfg.eps)
    assert_f16_close(to_bits(xn), O.rmsnorm_f16(to_bits(x), w_in.cpu().numpy(), cfg.eps), what="qwen3 chain rmsnorm in")

    _case("qwen3 chain: qkv projection")
    w_qkv, c_qkv = _onehot(QW, C, 7, 3, dev)
    qkv = _project(xn, w_qkv, C, c_qkv, "qkv")

    _case("qwen3 chain: q/k norm + rope + kv store, per sequence")
    qkv_in = to_bits(qkv).copy()
    kc = torch.empty((T // S, S, KVW), dtype=torch.float16, device=dev)
    vc = torch.empty_like(kc)
    for s in range(T // S):
        ops.qk_norm_rope_kv(qkv[s * S:(s + 1) * S], H, KV, hd, cs, cfg.eps, kc[s], vc[s], wqk=wqk)
    wqk_h = wqk.cpu().numpy()
    got = to_bits(qkv)
    for s in range(T // S):
        rows = slice(s * S, (s + 1) * S)
        want, wk, wv = O.qk_norm_rope_kv(qkv_in[rows], H, KV, hd, cs_host, S, cfg.eps, wqk=wqk_h)
        assert_f16_close(got[rows, :QH + KVW], want[:, :QH + KVW], what=f"qwen3 chain q/k rope seq {s}")
        assert np.array_equal(got[rows, QH + KVW:], qkv_in[rows, QH + KVW:]), "v heads were written"
        assert_f16_close(to_bits(kc[s]), wk, what=f"qwen3 chain k cache seq {s}")
        assert np.array_equal(to_bits(vc[s]), wv), f"v cache seq {s}"

    _case("qwen3 chain: attention over each sequence's caches")
    att = torch.empty((T, QH), dtype=torch.float16, device=dev)
    for s in range(T // S):
        rows = slice(s * S, (s + 1) * S)
        ops.attention(qkv[rows, :QH], kc[s], vc[s], H, KV, hd, 0, out=att[rows])
    got_att = att.float().cpu().numpy()
    rng = np.random.default_rng(9)
    for s in range(T // S):
        kb = to_bits(kc[s])
        vb = to_bits(vc[s])
        for t in sorted({0, 1, S - 1, *rng.integers(2, S - 1, 5).tolist()}):
            qrow = got[s * S + t:s * S + t + 1, :QH].view(np.float16).astype(np.float32)
            want = O.attention(qrow, kb[:t + 1], vb[:t + 1], H, KV, hd, t)[0]
            half_ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float32) / 2
            excess = np.abs(got_att[s * S + t] - want) - half_ulp - 2e-6 * (1.0 + np.abs(want))
            assert (excess <= 0).all(), f"qwen3 chain attention seq {s} token {t}"

    _case("qwen3 chain: o projection + residual add + rmsnorm")
    w_o, c_o = _onehot(C, QH, 3, 11, dev)
    delta = _project(att, w_o, QH, c_o, "o")
    x_in = to_bits(x).copy()
    xn2 = ops.add_rms_norm(x, delta, w_post, cfg.eps)
    want_x, want_xn = O.add_rmsnorm_f16(x_in, to_bits(delta), w_post.cpu().numpy(), cfg.eps)
    assert np.array_equal(to_bits(x), want_x), "residual sum"
    assert_f16_close(to_bits(xn2), want_xn, what="qwen3 chain add+rmsnorm")

    _case("qwen3 chain: gate/up projection + swiglu")
    w_gu, c_gu = _onehot(2 * F, C, 9, 5, dev)
    h = _project(xn2, w_gu, C, c_gu, "gate/up")
    g = ops.silu_mul(h)
    assert_f16_close(to_bits(g), O.swiglu_f16(to_bits(h)), what="qwen3 chain swiglu")

    _case("qwen3 chain: down projection accumulated into the residual")
    w_d, c_d = _onehot(C, F, 13, 1, dev)
    x_before = x.float()
    ops.matmul(g, w_d, ops.FMT_F16, F, out=x, flags=ops.MM_ACCUMULATE)
    want = (x_before + g.float()[:, torch.from_numpy(c_d).to(dev)]).half()  # f32 add, one RNE
    assert torch.equal(x, want), "down projection residual"


def test_granite_mamba_layer_chain(dev):
    """rmsNorm -> in_proj -> (Mamba scan stand-in) -> gated group RMSNorm in place with z read from
    the in_proj row -> out_proj -> residual add + rmsNorm -> gate/up projection -> SwiGLU; 16384
    tokens, hidden 1536, d_inner 3072, I = 4096."""
    cfg = wl.GRANITE_NORMS
    T, C, D, I = cfg.T, cfg.C, cfg.D, cfg.I
    P = 2 * D + 64  # in_proj row: z (the first D columns), then the rest of the projection
    x = wl.normal_f16((T, C), 0.0, 1.0, 21, "cpu").to(dev)
    w1 = wl.weight_f32(C, 1.0, 0.05, 22, "cpu").to(dev)
    wg = wl.weight_f32(D, 1.0, 0.05, 23, "cpu").to(dev)
    w2 = wl.weight_f32(C, 1.0, 0.05, 24, "cpu").to(dev)

    _case("granite chain: input rmsnorm")
    xn = ops.rms_norm(x, w1, cfg.eps)
    assert_f16_close(to_bits(xn), O.rmsnorm_f16(to_bits(x), w1.cpu().numpy(), cfg.eps), what="granite chain rmsnorm in")

    _case("granite chain: in_proj")
    w_in, c_in = _onehot(P, C, 5, 7, dev)
    proj = _project(xn, w_in, C, c_in, "in_proj")
    z = proj[:, :D]  # strided view: the gate columns of the in_proj row
    y = proj[:, D:2 * D].clone()  # stands in for the scan output y_

    _case("granite chain: gated group rmsnorm in place")
    want = O.gated_rmsnorm_f16(to_bits(y), np.ascontiguousarray(to_bits(z)), wg.cpu().numpy(), cfg.groups, cfg.eps)
    ops.gated_rms_norm(y, z, wg, cfg.groups, cfg.eps, out=y)
    assert_f16_close(to_bits(y), want, what="granite chain gated")

    _case("granite chain: out_proj + residual add + rmsnorm")
    w_out, c_out = _onehot(C, D, 11, 2, dev)
    delta = _project(y, w_out, D, c_out, "out_proj")
    x_in = to_bits(x).copy()
    xn2 = ops.add_rms_norm(x, delta, w2, cfg.eps)
    want_x, want_xn = O.add_rmsnorm_f16(x_in, to_bits(delta), w2.cpu().numpy(), cfg.eps)
    assert np.array_equal(to_bits(x), want_x), "residual sum"
    assert_f16_close(to_bits(xn2), want_xn, what="granite chain add+rmsnorm")

    _case("granite chain: gate/up projection + swiglu")
    w_gu, c_gu = _onehot(2 * I, C, 3, 9, dev)
    h = _project(xn2, w_gu, C, c_gu, "gate/up")
    assert_f16_close(to_bits(ops.silu_mul(h)), O.swiglu_f16(to_bits(h)), what="granite chain swiglu")
