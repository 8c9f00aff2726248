"""The five configured workloads: shapes, synthetic inputs and algorithmic byte counts.

Algorithmic bytes (the roofline numerator): fp16 activations read once and written once, f32 norm
weights once, int32 ids / positions counted, the gather counts per-token row bytes + output + ids;
V heads in the qkv buffer and the RoPE cos/sin table are not counted.

Inputs are drawn with torch's Philox generator (seed 0, one stream id per tensor), normals in f32
then rounded once to fp16; weights are rounded to fp16 (as a checkpoint would hold them) and kept as
f32. Token ids use numpy's PCG64 with the same seeding. Everything is deterministic for a given seed
and device (torch's CPU and GPU generators give different streams; tests draw on the CPU and copy).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch

SEED = 0


def _gen(stream: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(SEED * 1_000_003 + 7919 * stream + 1)
    return g


def normal_f16(shape, mean: float, std: float, stream: int, device) -> torch.Tensor:
    """~N(mean, std) rounded to fp16."""
    z = torch.randn(shape, generator=_gen(stream, device), device=device, dtype=torch.float32)
    return (z * std + mean).to(torch.float16)


def weight_f32(n: int, mean: float, std: float, stream: int, device) -> torch.Tensor:
    """Norm/gate weights: ~N(mean, std), fp16-rounded, stored f32 (the reference keeps f32 copies)."""
    return normal_f16((n,), mean, std, stream, device).to(torch.float32)


def uniform_ids(n: int, vocab: int, stream: int) -> np.ndarray:
    rng = np.random.default_rng([SEED, stream])
    return rng.integers(0, vocab, n, dtype=np.int64).astype(np.int32)


def zipf_ids(n: int, vocab: int, s: float, stream: int) -> np.ndarray:
    """ids = rank - 1 with P(rank) proportional to rank^-s over 1..vocab (inverse CDF)."""
    rng = np.random.default_rng([SEED, stream])
    p = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int32)


# ------------------------------------------------------------------ byte counts

def bytes_rmsnorm(T: int, C: int, e: int = 2) -> int:
    """x read and y written (e-byte activations: 2 for f16, 4 for f32), the f32 weights once."""
    return 2 * T * C * e + C * 4


def bytes_layernorm(T: int, C: int) -> int:
    return 2 * T * C * 2 + 2 * C * 4


def bytes_qk_rope(T: int, n_q: int, n_kv: int, hd: int, positions: bool = True, e: int = 2) -> int:
    return 2 * T * (n_q + n_kv) * hd * e + (T * 4 if positions else 0) + 2 * hd * 4


def bytes_swiglu(T: int, I: int, e: int = 2) -> int:
    return T * (2 * I * e + I * e)


def bytes_gelu(n: int) -> int:
    return 2 * n * 2


def bytes_gated(T: int, D: int) -> int:
    return 3 * T * D * 2 + D * 4


def bytes_gather(T: int, row_bytes: int, C: int, wpe: bool = False) -> int:
    return T * (row_bytes + C * 2 + 4 + (C * 2 if wpe else 0))


def bytes_add_rmsnorm(T: int, C: int) -> int:
    """x and delta read, x and xn written (fp16), the weights once."""
    return 4 * T * C * 2 + C * 4


def bytes_store_kv(T: int, width: int, positions: bool = True) -> int:
    """k and v read (fp16), both written to the caches, plus the positions."""
    return 4 * T * width * 2 + (T * 4 if positions else 0)


def bytes_matmul(T: int, K: int, N: int, row_bytes: int, y_bytes: int = 4, accumulate: bool = False,
                 x_bytes: int = 2) -> int:
    """The weight rows read once, the activations (x_bytes each) read, the outputs written (and read
    when accumulating)."""
    return N * row_bytes + T * K * x_bytes + T * N * y_bytes * (2 if accumulate else 1)


def bytes_qk_rope_kv(T: int, n_q: int, n_kv: int, hd: int, positions: bool = True) -> int:
    """q/k RoPE bytes plus the v heads read and the k and v heads written to the caches."""
    return bytes_qk_rope(T, n_q, n_kv, hd, positions) + 3 * T * n_kv * hd * 2


# ------------------------------------------------------------------ configurations

@dataclasses.dataclass(frozen=True)
class Qwen3Prefill:
    """Qwen3-4B-shaped prefill: 4 x 2048 tokens, hidden 2560, 32 q + 8 kv heads of 128, I = 9728."""
    T: int = 8192
    C: int = 2560
    n_q: int = 32
    n_kv: int = 8
    hd: int = 128
    I: int = 9728
    seq: int = 2048
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def qkv_stride(self) -> int:
        return (self.n_q + 2 * self.n_kv) * self.hd

    def op_bytes(self) -> dict:
        rms = bytes_rmsnorm(self.T, self.C)
        return {
            "rmsnorm_in": rms,
            "qk_norm_rope": bytes_qk_rope(self.T, self.n_q, self.n_kv, self.hd),
            "rmsnorm_post": rms,
            "swiglu": bytes_swiglu(self.T, self.I),
        }


@dataclasses.dataclass(frozen=True)
class Qwen3Decode:
    """Qwen3-0.6B-shaped decode batch: 64 rows, hidden 1024, 16 q + 8 kv heads of 128, I = 3072."""
    T: int = 64
    C: int = 1024
    n_q: int = 16
    n_kv: int = 8
    hd: int = 128
    I: int = 3072
    n_pos: int = 4096
    eps: float = 1e-6
    theta: float = 1e6


@dataclasses.dataclass(frozen=True)
class Gpt2Chain:
    """GPT-2 small layer-op chain: T = 128, C = 768, wte 50257 x 768, wpe 1024 x 768, GELU on 3072."""
    T: int = 128
    C: int = 768
    vocab: int = 50257
    n_ctx: int = 1024
    F: int = 3072
    eps: float = 1e-5


@dataclasses.dataclass(frozen=True)
class QuantGather:
    """Qwen3-1.7B-shaped tied table 151936 x 2048, 16384 Zipf(1.1) ids."""
    vocab: int = 151936
    C: int = 2048
    T: int = 16384
    s: float = 1.1


@dataclasses.dataclass(frozen=True)
class Qwen3DecodeMatmul:
    """Qwen3-4B decode: the layer's four weight matmuls for T tokens (one decode step of T sequences):
    q/k/v [6144, 2560], o [2560, 4096], gate/up [19456, 2560], down [2560, 9728]."""
    T: int = 1
    projections: tuple = (("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560), ("down", 2560, 9728))


@dataclasses.dataclass(frozen=True)
class Qwen3PrefillMatmul:
    """Qwen3-4B prefill: the layer's four weight matmuls over 4 x 2048 = 8192 tokens."""
    T: int = 8192
    projections: tuple = (("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560), ("down", 2560, 9728))


@dataclasses.dataclass(frozen=True)
class GraniteNorms:
    """Granite-4.0-H-style: 16384 tokens, RMSNorm over 1536, gated norm over d_inner 3072, SwiGLU I = 4096."""
    T: int = 16384
    C: int = 1536
    D: int = 3072
    groups: int = 1
    I: int = 4096
    eps: float = 1e-5


QWEN3_PREFILL = Qwen3Prefill()
QWEN3_DECODE = Qwen3Decode()
GPT2_CHAIN = Gpt2Chain()
QUANT_GATHER = QuantGather()
GRANITE_NORMS = GraniteNorms()
QWEN3_DECODE_MATMUL = Qwen3DecodeMatmul()
QWEN3_DECODE4_MATMUL = Qwen3DecodeMatmul(T=4)  # one decode step of 4 sequences
QWEN3_DECODE16_MATMUL = Qwen3DecodeMatmul(T=16)  # one decode step of 16 sequences
QWEN3_DECODE24_MATMUL = Qwen3DecodeMatmul(T=24)  # one decode step of 24 sequences
QWEN3_PREFILL_MATMUL = Qwen3PrefillMatmul()


def qwen3_prefill_inputs(cfg: Qwen3Prefill, device) -> dict:
    """Synthetic inputs for one Qwen3-4B prefill layer's non-GEMM ops (all resident on `device`)."""
    from . import ops  # host codecs only
    pos = (np.arange(cfg.T) % cfg.seq).astype(np.int32)
    return {
        "x": normal_f16((cfg.T, cfg.C), 0.0, 1.0, 1, device),
        "w_in": weight_f32(cfg.C, 1.0, 0.05, 2, device),
        "w_post": weight_f32(cfg.C, 1.0, 0.05, 3, device),
        "x_post": normal_f16((cfg.T, cfg.C), 0.0, 1.0, 7, device),  # the post-attention residual
        "qkv": normal_f16((cfg.T, cfg.qkv_stride), 0.0, 1.0, 4, device),
        "wqk": weight_f32(2 * cfg.hd, 1.0, 0.05, 5, device),
        "positions": torch.from_numpy(pos).to(device),
        "cs": torch.from_numpy(ops.rope_table(cfg.theta, cfg.hd, cfg.seq)).to(device),
        "h": normal_f16((cfg.T, 2 * cfg.I), 0.0, 1.0, 6, device),
    }
