"""Weight tables for the matmul tests, written directly in the reference's row layout (quant.h:30-36):
F16 rows of K halves; FP8 rows of K E4M3 codes then K/32 f16 block scales, padded to 16 bytes; FP4 rows
of K/32 16-byte blocks (weight j of a block in the low nibble of byte j, weight 16 + j in its high
nibble) then the scales, padded likewise.

`integer_table` builds rows whose dequantised values are small integers (codes of integers times
power-of-two scales), so with integer activations every product and every partial sum is an exact
float and any summation order gives the same bits.
"""
import numpy as np

from oracle import oracle as O

F16_ONE = 0x3C00


def _f16_bits(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def row_bytes(fmt, K):
    return int(O.lib().oracle_quant_row_bytes(fmt, K))


def pack_rows(fmt, codes, scales):
    """codes: [N, K] uint8 (FP8 codes / FP4 nibbles) or uint16 f16 bits (F16); scales: [N, K/32] f16 bits."""
    N, K = codes.shape
    rb = row_bytes(fmt, K)
    out = np.zeros((N, rb), np.uint8)
    if fmt == O.FMT_F16:
        out[:, :2 * K] = np.ascontiguousarray(codes, np.uint16).view(np.uint8)
        return out
    nb = K // 32
    if fmt == O.FMT_FP8:
        out[:, :K] = codes
        soff = K
    else:
        c = codes.reshape(N, nb, 32).astype(np.uint8)
        out[:, :K // 2] = (c[:, :, :16] | (c[:, :, 16:] << 4)).reshape(N, K // 2)
        soff = K // 2
    out[:, soff:soff + 2 * nb] = np.ascontiguousarray(scales, np.uint16).view(np.uint8).reshape(N, 2 * nb)
    return out


def integer_table(fmt, N, K, rng):
    """(table, dense float32 weights): integer weights in [-8, 8] (F16, FP8) or {0, +-1..12} (FP4)."""
    nb = K // 32 if fmt != O.FMT_F16 else 0
    if fmt == O.FMT_F16:
        w = rng.integers(-8, 9, (N, K)).astype(np.float32)
        return pack_rows(fmt, _f16_bits(w), None), w
    L = O.lib()
    if fmt == O.FMT_FP8:
        vals = rng.integers(-8, 9, (N, K)).astype(np.float32)
        scale_pow = rng.integers(0, 2, (N, nb))  # scale 1 or 2
        scales = (2.0 ** scale_pow).astype(np.float32)
        codes = np.array([L.oracle_encode_fp8(float(v)) for v in range(-8, 9)], np.uint8)[(vals + 8).astype(int)]
    else:
        grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float32)
        idx = rng.integers(0, 8, (N, K))
        sign = rng.integers(0, 2, (N, K))
        vals = grid[idx] * np.where(sign == 1, -1.0, 1.0).astype(np.float32)
        codes = (idx | (sign << 3)).astype(np.uint8)
        scale_pow = rng.integers(1, 3, (N, nb))  # scale 2 or 4: every value an integer
        scales = (2.0 ** scale_pow).astype(np.float32)
    w = vals * np.repeat(scales, 32, axis=1)
    return pack_rows(fmt, codes, _f16_bits(scales)), w.astype(np.float32)


def dequant(fmt, table, K):
    """The oracle's dequantisation of every row: float32 [N, K]."""
    out = np.empty((table.shape[0], K), np.float32)
    for r in range(table.shape[0]):
        O.lib().oracle_dequantize_row(fmt, K, O._ptr(table[r]), O._ptr(out[r]))
    return out


def exact_and_bound(x, w, bias=None):
    """float64 x . w^T (+ bias) and sum_k |x_k w_k| (+ |bias|), the scale of any f32 summation error."""
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    exact = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    if bias is not None:
        exact = exact + bias.astype(np.float64)
        mag = mag + np.abs(bias.astype(np.float64))
    return exact, mag


def qwen3_table_source(vocab=151936, cols=2048):
    """The Qwen3-1.7B-shaped tied embedding table in f32, ~N(0, 0.02) from numpy's PCG64 (seed [0, 41]):
    identical on every machine, so its encoded tables can be pinned by sha256."""
    rng = np.random.default_rng([0, 41])
    x = rng.standard_normal((vocab, cols), dtype=np.float32)
    x *= np.float32(0.02)
    return x
