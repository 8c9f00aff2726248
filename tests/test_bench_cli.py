"""bench.py's command line without a GPU: it parses, lists its workloads, and refuses more than one GPU
before touching a device (N > 1 exits with a message)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_help_lists_every_workload():
    r = _run("--help")
    assert r.returncode == 0, r.stderr
    text = " ".join(r.stdout.split())
    for w in ("gpt2_small_chain", "qwen3_0.6b_decode", "qwen3_4b_prefill", "qwen3_4b_prefill_f32", "quant_gather_qwen3_1.7b",
              "qwen3_4b_fused",
              "quantize_qwen3_1.7b_table", "granite_4.0h_norms", "qwen3_4b_decode_matmul", "qwen3_4b_decode4_matmul",
              "qwen3_4b_decode16_matmul", "qwen3_4b_decode24_matmul", "qwen3_4b_decode_matmul_f32",
              "qwen3_4b_decode16_matmul_f32", "qwen3_4b_prefill_matmul"):
        assert w in text, w


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_floor_library_exports_what_bench_binds():
    """The streaming-floor kernels bench.py times beside the ops: every neko_floor_* function it binds is
    exported by the built libneko_floor.so (loaded without touching a device)."""
    import ctypes
    import re

    names = sorted(set(re.findall(r'"(neko_floor_[a-z0-9_]+)"', open(os.path.join(ROOT, "bench.py")).read())))
    assert "neko_floor_inplace_rows" in names and len(names) >= 6
    lib = ctypes.CDLL(os.path.join(ROOT, "nekochat_amd", "libneko_floor.so"))
    for n in names:
        assert hasattr(lib, n), f"bench.py binds {n}, which libneko_floor.so does not export"


def test_floor_calls_declare_their_argument_types():
    """bench.FloorLib hands out only floor functions whose ctypes argument types it declares (without
    them, 64-bit device pointers would be passed as truncated 32-bit ints), and declares one for every
    function the floor library exports. Checked without a device: the library loads on the CPU."""
    import ctypes
    import re
    import subprocess as sp

    sys.path.insert(0, ROOT)
    import bench

    fl = bench.FloorLib.__new__(bench.FloorLib)
    bench.FloorLib.__init__(fl, 0)
    out = sp.run(["nm", "-D", "--defined-only", os.path.join(ROOT, "nekochat_amd", "libneko_floor.so")],
                 capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(neko_floor_[a-z0-9_]+)\b", out))
    assert exported and exported == fl.bound, (exported, fl.bound)
    for name in fl.bound:
        assert getattr(fl.lib, name).argtypes, name
    try:
        fl.not_a_function
    except AttributeError:
        pass
    else:
        raise AssertionError("FloorLib returned a function without declared argument types")
    del ctypes
