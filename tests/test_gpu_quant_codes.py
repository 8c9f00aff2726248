"""The device quantiser's FP4 / FP8 codes come from gfx950's E2M1 / E4M3 conversion instructions with
corrections (nekochat_amd/csrc/quant_codes.h). tests/cpp/quant_codes_check.hip compares them with the
reference quantiser's own arithmetic (quant.cpp:43-49, 57-61, 93-97) over every f32 bit pattern."""
import ctypes
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(HERE, "cpp", "_build", "libquant_codes_check.so")


@pytest.mark.gpu
def test_quant_codes_every_f32_pattern(dev):
    print("[case] quantiser conversion codes over every f32 pattern", flush=True)
    if not os.path.exists(HARNESS):
        pytest.fail(f"{HARNESS} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(HARNESS)
    lib.neko_test_quant_codes.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint32)]
    lib.neko_test_quant_codes.restype = ctypes.c_int
    counts = (ctypes.c_ulonglong * 6)()
    first = (ctypes.c_uint32 * 3)()
    assert lib.neko_test_quant_codes(counts, first) == 0
    c = list(counts)
    # fp4 rounding (2^31 non-negative patterns) and fp4 encode (2^32): every pattern, NaN included
    assert c[0] == 0 and c[1] == 0, f"fp4 rounding differs on {c[0]} + {c[1]} (NaN) patterns, first {first[0]:#010x}"
    assert c[2] == 0 and c[3] == 0, f"fp4 encode differs on {c[2]} + {c[3]} (NaN) patterns, first {first[1]:#010x}"
    # fp8 encode: every non-NaN pattern (NaN weights are outside the quantiser's pinned inputs)
    assert c[4] == 0, f"fp8 encode differs on {c[4]} non-NaN patterns, first {first[2]:#010x}"
