"""GPU causal grouped-query attention (neko_hip_attention) against the oracle's restatement of
cpu::attention (cpu_ops.cpp:544-575), which tests/test_oracle.py pins bit-exact to the compiled
reference and to a float64 softmax.

No canonical summation order exists -- the reference's CPU loop and its shader (attention.comp) sum
in different orders -- so the bar is a tolerance, written below: |gpu - oracle| <= TOL * (1 + |oracle|)
with TOL = 2e-6 for f32 outputs (the reference's own self-test allows 2e-3), and f16 outputs within
half an f16 ulp of the oracle's f32 result plus that bar. Shapes: the reference self-test case, the Qwen3-4B
decode (one token over 4096 and 40000 cached positions: the keys split over many workgroups and
merged; one kv head over 100000 positions: 391 splits) and a 256-token prefill, GPT-2 heads, head
sizes 6 / 96 / 256 (the per-half and masked loads), groups of 3 and 8 query heads per kv head, work
items of one and of four query heads, strided q / out rows, f16 activations, and the argument checks.
"""
import numpy as np
import pytest
import torch

from nekochat_amd import NekoError, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-6


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _inputs(T, H, KV, hd, pos0, dev, seed, q_extra=0, dtype=torch.float32):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn((T, H * hd + q_extra), generator=g, dtype=torch.float32)
    kc = torch.randn((pos0 + T, KV * hd), generator=g, dtype=torch.float32).half()
    vc = torch.randn((pos0 + T, KV * hd), generator=g, dtype=torch.float32).half()
    if dtype == torch.float16:
        q = q.half()
    return q.to(dev), kc.to(dev), vc.to(dev)


def _oracle(q, kc, vc, H, KV, hd, pos0):
    qf = q.float().cpu().numpy()
    return O.attention(qf, kc.cpu().view(torch.int16).numpy().view(np.uint16),
                       vc.cpu().view(torch.int16).numpy().view(np.uint16), H, KV, hd, pos0)


def _check_f32(got, want, what):
    got = got.cpu().numpy()
    err = np.abs(got - want) / (1.0 + np.abs(want))
    worst = float(err.max())
    print(f"{what}: worst |gpu - oracle| / (1 + |oracle|) = {worst:.3e}", flush=True)
    assert np.isfinite(got).all(), what
    assert worst <= TOL, f"{what}: {worst:.3e} > {TOL}"


@pytest.mark.parametrize("T,H,KV,hd,pos0", [
    (3, 4, 2, 64, 1030),    # the reference self-test case (compute.cpp:262-283)
    (1, 32, 8, 128, 4095),  # Qwen3-4B decode, 4096 cached positions: keys split over waves
    (4, 32, 8, 128, 2000),  # four-sequence decode step
    (256, 32, 8, 128, 0),   # Qwen3-4B prefill of 256 tokens: one item per (token, kv head)
    (64, 12, 12, 64, 0),    # GPT-2 small: one query head per kv head
    (8, 8, 2, 256, 100),    # head size 256, one query head per work item
    (512, 8, 2, 256, 0),    # head size 256, four query heads per work item
    (5, 6, 2, 96, 70),      # head size 96: dimensions past hd masked
    (3, 4, 2, 6, 9),        # head size 6: per-half loads, one query head per work item
    (512, 4, 2, 6, 0),      # head size 6, two query heads per work item
    (7, 12, 4, 64, 200),    # three query heads per kv head
    (2, 16, 2, 128, 3000),  # eight query heads per kv head, one per work item
    (1, 16, 2, 128, 40000),  # eight query heads per kv head: two blocks of four (41 MB of K and V)
    (1, 32, 8, 128, 40000),  # long context: 126 splits merged
    (1, 4, 1, 128, 100000),  # one kv head: 391 splits (the merge's threads each take several)
])
def test_attention_f32(dev, T, H, KV, hd, pos0):
    _case(f"attention f32 T={T} H={H} KV={KV} hd={hd} pos0={pos0}")
    q, kc, vc = _inputs(T, H, KV, hd, pos0, dev, seed=T * 131 + hd + pos0)
    out = ops.attention(q, kc, vc, H, KV, hd, pos0)
    torch.cuda.synchronize()
    _check_f32(out, _oracle(q, kc, vc, H, KV, hd, pos0), f"attention T={T} H={H} KV={KV} hd={hd} pos0={pos0}")


def test_attention_strided_rows(dev):
    """q as the first columns of qkv rows (the models' layout) and out rows wider than n_head*hd."""
    _case("attention strided q / out rows")
    T, H, KV, hd, pos0 = 9, 8, 2, 64, 33
    qkv, kc, vc = _inputs(T, H, KV, hd, pos0, dev, seed=7, q_extra=2 * KV * hd)
    q = qkv[:, : H * hd]
    out_full = torch.full((T, H * hd + 40), 7.0, dtype=torch.float32, device=dev)
    out = out_full[:, : H * hd]
    ops.attention(q, kc, vc, H, KV, hd, pos0, out=out)
    torch.cuda.synchronize()
    _check_f32(out, _oracle(q, kc, vc, H, KV, hd, pos0), "attention strided")
    assert torch.all(out_full[:, H * hd:] == 7.0), "columns past n_head*hd were written"


def test_attention_f16(dev):
    """f16 q and out: the oracle's f32 result of the same (f16-valued) q, within half an f16 ulp (the
    rounding) plus the f32 bar above."""
    _case("attention f16")
    T, H, KV, hd, pos0 = 16, 32, 8, 128, 500
    q, kc, vc = _inputs(T, H, KV, hd, pos0, dev, seed=11, dtype=torch.float16)
    out = ops.attention(q, kc, vc, H, KV, hd, pos0)
    torch.cuda.synchronize()
    want = _oracle(q, kc, vc, H, KV, hd, pos0)
    got = out.float().cpu().numpy()
    half_ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float32) / 2
    excess = np.abs(got - want) - half_ulp - TOL * (1.0 + np.abs(want))
    print(f"attention f16: worst excess over half an ulp + bar = {excess.max():.3e}", flush=True)
    assert (excess <= 0).all()


def test_attention_scale_and_single_key(dev):
    """Position 0 sees one key: out = v_0 exactly, whatever q or the scale. A zero scale weights every
    key alike: out = the mean of the v rows."""
    _case("attention single key / zero scale")
    H, KV, hd = 4, 2, 64
    q, kc, vc = _inputs(1, H, KV, hd, 0, dev, seed=3)
    out = ops.attention(q, kc, vc, H, KV, hd, 0, scale=0.37)
    torch.cuda.synchronize()
    want = torch.cat([vc[0, (h // 2) * hd:(h // 2 + 1) * hd] for h in range(H)]).float()
    assert torch.equal(out[0], want)
    T, pos0 = 2, 300
    q, kc, vc = _inputs(T, H, KV, hd, pos0, dev, seed=4)
    out = ops.attention(q, kc, vc, H, KV, hd, pos0, scale=0.0)
    torch.cuda.synchronize()
    v = vc.double().cpu()
    for t in range(T):
        mean = v[: pos0 + t + 1].mean(0)
        want = torch.cat([mean[(h // 2) * hd:(h // 2 + 1) * hd] for h in range(H)])
        assert torch.allclose(out[t].double().cpu(), want, rtol=0, atol=1e-5)


def test_attention_argument_checks(dev):
    _case("attention argument checks")
    q, kc, vc = _inputs(2, 4, 2, 64, 5, dev, seed=5)
    assert ops.attention(q[:0], kc, vc, 4, 2, 64, 5).shape == (0, 256)  # no tokens: nothing to do
    with pytest.raises(NekoError):
        ops.attention(q, kc, vc, 3, 2, 64, 5)  # n_head not a multiple of n_kv
    with pytest.raises(NekoError):
        ops.attention(q, kc[:6], vc, 4, 2, 64, 5)  # caches shorter than pos0 + T
    qo, kco, vco = _inputs(2, 4, 2, 63, 5, dev, seed=6)
    with pytest.raises(NekoError):
        ops.attention(qo, kco, vco, 4, 2, 63, 5)  # odd head size
    with pytest.raises(NekoError):
        ops.attention(q, kc, vc, 4, 2, 64, 5, out=q)  # out over q
