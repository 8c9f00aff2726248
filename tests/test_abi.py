"""The C-ABI library without a GPU: it loads, exports every function include/neko_hip.h declares, fails
cleanly where no device is present, and its host-side codecs (quantizeMatrix, ropeTable, quantRowBytes
equivalents) are bit-identical to the oracle and, where built, the compiled reference."""
import ctypes
import os
import re

import numpy as np
import pytest

from nekochat_amd import _lib, ops
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "neko_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(neko_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(_lib.lib, n), f"{n} declared in include/neko_hip.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert sorted(_lib.SIGNATURES) == names


def _has_gpu():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_create_without_device_fails_cleanly():
    h = ctypes.c_void_p(123)
    rc = _lib.lib.neko_hip_create(0, ctypes.byref(h))
    assert rc == _lib.NEKO_ERR_NO_DEVICE
    assert h.value is None
    assert b"device" in _lib.lib.neko_hip_last_error(None)
    with pytest.raises(_lib.NekoError):
        ops.Context(0)


def test_null_context_is_rejected_without_touching_a_device():
    L = _lib.lib
    assert L.neko_hip_rmsnorm(None, None, 0, None, 0, None, 4, 8, 1e-6, 1) == _lib.NEKO_ERR_INVALID
    assert L.neko_hip_swiglu(None, None, 0, None, 0, 1, 8, 1) == _lib.NEKO_ERR_INVALID
    assert L.neko_hip_embed(None, None, 1, None, 64, 0, 32, 0, 1, None, 0, 0, None, 32, 1) == _lib.NEKO_ERR_INVALID
    assert L.neko_hip_last_error(None)
    assert L.neko_hip_destroy(None) == _lib.NEKO_OK
    assert L.neko_hip_get_stream(None) is None


def test_backend_factory_without_device():
    """createHip returns nullptr plus a message when no device opens (factory convention, vk_compute.cpp:459-466)."""
    if _has_gpu():
        pytest.skip("checks the no-device path")
    path = os.path.join(ROOT, "tests", "cpp", "_build", "libbackend_selftest.so")
    lib = ctypes.CDLL(path)
    lib.backend_create_without_device.argtypes = [ctypes.c_char_p, ctypes.c_int]
    buf = ctypes.create_string_buffer(512)
    assert lib.backend_create_without_device(buf, 512) == 0
    assert b"HIP" in buf.value


@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("cols", [32, 256, 2048, 100])
def test_host_quantizer_matches_oracle(fmt, cols):
    rng = np.random.default_rng(cols + fmt)
    x = (rng.standard_normal((97, cols)) * 0.02).astype(np.float32)
    x[1, :] = 0
    x[2, 7] = 2.5
    x[3, :] = rng.standard_t(1.5, cols) * 0.01
    want = O.quantize_rows(fmt, x)
    for threads in (1, 3, 0):
        got, used = ops.quantize_rows(fmt, x, threads=threads)
        assert used == (fmt if cols % 32 == 0 else 0)
        assert np.array_equal(got, want)
    if O.ref_available():
        ref = np.zeros_like(want)
        O.ref().ref_quantize_rows(fmt, 97, cols, O._ptr(x), O._ptr(ref))
        assert np.array_equal(got, ref)


def test_host_quant_row_bytes():
    for fmt in (0, 1, 2):
        for cols in (32, 64, 768, 1024, 2048, 3072):
            assert ops.quant_row_bytes(fmt, cols) == O.quant_row_bytes(fmt, cols)


def test_host_rope_table_matches_oracle():
    for theta, hd, n in ((1e6, 128, 4096), (1e4, 64, 100), (5e5, 256, 33)):
        assert np.array_equal(ops.rope_table(theta, hd, n).view(np.uint32), O.rope_table(theta, hd, n).view(np.uint32))


def test_host_codec_argument_errors():
    L = _lib.lib
    assert L.neko_quantize_rows(7, 1, 32, None, None, 1, None) == _lib.NEKO_ERR_INVALID
    assert L.neko_quantize_rows(1, 1, 32, None, None, 1, None) == _lib.NEKO_ERR_INVALID
    assert L.neko_rope_table(1e4, 3, 4, None) == _lib.NEKO_ERR_INVALID
    assert L.neko_quant_row_bytes(9, 32) == 0


def test_kernel_sources_carry_no_build_time_variants():
    """Every kernel source compiles one way: no NEKO_TUNE_* build-time switches whose other values no
    build compiles or tests (measured alternatives are recorded as measurements, not kept as code)."""
    import glob
    import re

    found = []
    for path in sorted(glob.glob(os.path.join(ROOT, "nekochat_amd", "csrc", "*"))):
        if not path.endswith((".hip", ".h", ".cpp", "Makefile")):
            continue
        for i, line in enumerate(open(path), 1):
            if re.search(r"\bNEKO_TUNE_\w+", line):
                found.append(f"{os.path.basename(path)}:{i}: {line.strip()}")
    assert not found, "\n".join(found)
