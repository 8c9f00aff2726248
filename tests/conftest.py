import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests of the HIP kernels")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU (run with -m 'not gpu' here)")
    return torch.device("cuda:0")


def f16_line(bits):
    """fp16 bit patterns -> integers on a monotone line (adjacent floats differ by 1; +0 == -0)."""
    b = np.asarray(bits).view(np.uint16).astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def f32_line(bits):
    b = np.asarray(bits, dtype=np.float32).view(np.uint32).astype(np.int64)
    return np.where(b & 0x80000000, -(b & 0x7FFFFFFF), b)


def ulp_diff_f16(got, want):
    """Per-element distance in fp16 units in the last place; NaN positions must match."""
    g = np.asarray(got).view(np.uint16)
    w = np.asarray(want).view(np.uint16)
    gn = (g & 0x7C00) == 0x7C00
    gn &= (g & 0x03FF) != 0
    wn = (w & 0x7C00) == 0x7C00
    wn &= (w & 0x03FF) != 0
    assert np.array_equal(gn, wn), "NaN positions differ"
    d = np.abs(f16_line(g) - f16_line(w))
    d[gn] = 0
    return d


PARITY = []  # (what, differing outputs, outputs, worst ulp) of every fp16 comparison this session


def assert_f16_close(got, want, max_ulp=2, what="", max_diff_frac=1e-3):
    """The fp16 parity bar: every output within max_ulp fp16 ulp of the oracle (2 = the stated bound),
    and at most max_diff_frac of the outputs not bit-identical (NaNs aside, whose positions must
    match). The kernels round where the reference rounds, so differences come only from summation
    order or the fast SiLU forms. None disables the second check."""
    d = ulp_diff_f16(got, want)
    worst = int(d.max()) if d.size else 0
    g = np.asarray(got).view(np.uint16)
    w = np.asarray(want).view(np.uint16)
    nan = ((w & 0x7C00) == 0x7C00) & ((w & 0x03FF) != 0)
    n = int(np.count_nonzero((g != w) & ~nan))  # bit patterns, so +0 vs -0 counts as a difference
    PARITY.append((what, n, int(d.size), worst))
    assert worst <= max_ulp, f"{what}: max {worst} fp16 ulp from the oracle ({n} of {d.size} differ)"
    if max_diff_frac is not None and d.size:
        assert n <= max_diff_frac * d.size, f"{what}: {n} of {d.size} outputs differ from the oracle"
    return d


def pytest_terminal_summary(terminalreporter):
    if not PARITY:
        return
    terminalreporter.write_sep("-", "fp16 parity against the oracle (outputs not bit-identical / total, worst ulp)")
    for what, n, size, worst in PARITY:
        terminalreporter.write_line(f"{what}: {n} / {size} ({n / max(size, 1):.2e}), worst {worst} ulp")


def to_bits(t):
    """A torch fp16 tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().cpu().contiguous().numpy().view(np.uint16)
