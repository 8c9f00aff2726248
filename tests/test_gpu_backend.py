"""The reference's backend self-test cases (gpu/compute.cpp:106-260, hot-path kernels) run through the
C++ HipBackend adapter with the reference's own dispatch parameter blocks (tests/cpp/backend_selftest.cpp)."""
import ctypes
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(HERE, "cpp", "_build", "libbackend_selftest.so")


def _harness():
    if not os.path.exists(HARNESS):
        pytest.fail(f"{HARNESS} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(HARNESS)
    for name in ("backend_selftest", "backend_create_without_device"):
        getattr(lib, name).argtypes = [ctypes.c_char_p, ctypes.c_int]
        getattr(lib, name).restype = ctypes.c_int
    return lib


@pytest.mark.gpu
def test_backend_selftest(dev):
    print("[case] HipBackend self-test", flush=True)
    buf = ctypes.create_string_buffer(1024)
    rc = _harness().backend_selftest(buf, 1024)
    assert rc == 0, buf.value.decode()
