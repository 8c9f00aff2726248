"""INTEGRATION.md's code examples compile against this repository's headers, so they cannot drift
from the adapter they describe (CPU only: g++ / gcc -fsyntax-only).

- The enum / factory declaration a maintainer adds to the reference's compute.h must number every
  kernel as nekochat_amd/csrc/compute.h does.
- Each `run(Kernel::..., {...}, gx, gy)` dispatch is compiled inside a function that declares `run`
  exactly as the reference's models do (qwen3_model.cpp:288-294: the parameters travel as a
  std::initializer_list<int32_t>), so a float passed where the adapter decodes float bits
  (`bitsFloat(pa[1])`, hip_backend.cpp) is a narrowing error, not a silently garbled eps.
- The C example compiles as C11 against include/neko_hip.h.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")


def _blocks(lang):
    text = open(DOC).read()
    return re.findall(r"```" + lang + r"\n(.*?)```", text, flags=re.S)


def _compile(tmp_path, name, source, compiler, flags):
    path = tmp_path / name
    path.write_text(source)
    r = subprocess.run([compiler, *flags, "-fsyntax-only", str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"{name} does not compile:\n{source}\n{r.stderr}"
    return r


CPP_PRELUDE = r"""
#include <cstdint>
#include <initializer_list>
#include "compute.h"
using namespace neko::gpu;
// What the reference's model code has in scope at its dispatch sites (qwen3_model.cpp:280-317,
// granite_model.h:31-40).
struct Layer { Buffer *wqkv, *bqkv, *norm, *ln2, *kCache, *vCache; };
struct Config { float eps; int mGroups; float embeddingMult; };
void dispatches(ComputeBackend& be, Layer L, Config cfg_, Buffer* xn, Buffer* qkv, Buffer* y, Buffer* proj, Buffer* x,
                Buffer* d, int C, int QW, int T, int DI, int P, float eps, Buffer* tokens, Buffer* table, int flags,
                int rows, int rowWords, Buffer* gQkv_, Buffer* gAtt_, int H, int pos0, int hd, int32_t scale, int KW) {
    auto run = [&](Kernel k, Buffer* a, Buffer* b, Buffer* c, Buffer* e, std::initializer_list<int32_t> p, uint32_t gx,
                   uint32_t gy) {
        Buffer* binds[4] = {a, b, c, e};
        int32_t params[8] = {};
        int i = 0;
        for (int32_t v : p) params[i++] = v;
        be.dispatch(k, binds, params, gx, gy);
    };
    (void)xn; (void)qkv; (void)y; (void)proj; (void)x; (void)d; (void)C; (void)QW; (void)T; (void)DI; (void)P;
    (void)eps; (void)L; (void)cfg_; (void)tokens; (void)table; (void)flags; (void)rows; (void)rowWords;
    (void)gQkv_; (void)gAtt_; (void)H; (void)pos0; (void)hd; (void)scale; (void)KW;
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_cpp_dispatch_snippets_compile(tmp_path):
    runs = []
    for block in _blocks("cpp"):
        runs += [ln for ln in block.splitlines() if ln.strip().startswith("run(Kernel::")]
    assert len(runs) >= 3, "INTEGRATION.md lost its dispatch examples"
    body = "\n".join("    " + ln.strip() for ln in runs)
    src = CPP_PRELUDE + body + "\n}\n"
    _compile(tmp_path, "dispatch.cpp", src, "g++",
             ["-std=c++17", "-Wall", "-Werror", "-Werror=narrowing", "-I", os.path.join(ROOT, "nekochat_amd", "csrc")])


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_cpp_narrowing_is_caught(tmp_path):
    """The harness rejects the mistake it exists for: a raw float eps in the parameter block."""
    src = CPP_PRELUDE + "    run(Kernel::GatedRmsNorm, y, proj, L.norm, nullptr, {DI, cfg_.eps, cfg_.mGroups, P}, 1, 1);\n}\n"
    path = tmp_path / "bad.cpp"
    path.write_text(src)
    r = subprocess.run(["g++", "-std=c++17", "-Werror=narrowing", "-fsyntax-only", "-I",
                        os.path.join(ROOT, "nekochat_amd", "csrc"), str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "narrowing" in r.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_enum_snippet_matches_compute_h(tmp_path):
    decl = next(b for b in _blocks("cpp") if "enum class Kernel" in b)
    enum = re.search(r"enum class Kernel[^{]*\{(.*?)\};", decl, flags=re.S)
    assert enum, "INTEGRATION.md lost the Kernel enum"
    names = [n.split("=")[0].strip() for n in enum.group(1).split(",") if n.strip()]
    checks = "\n".join(f"static_assert(int(doc::Kernel::{n}) == int(neko::gpu::Kernel::{n}), \"{n}\");" for n in names)
    src = ("#include <memory>\n#include <string>\n#include \"compute.h\"\nnamespace doc {\n"
           "struct ComputeBackend;\n" + decl.replace("std::unique_ptr<ComputeBackend> createHip",
                                                     "std::unique_ptr<neko::gpu::ComputeBackend> createHip") +
           "\n}\n" + checks + "\n")
    _compile(tmp_path, "enum.cpp", src, "g++", ["-std=c++17", "-Wall", "-I", os.path.join(ROOT, "nekochat_amd", "csrc")])


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c_snippet_compiles(tmp_path):
    block = next(b for b in _blocks("c") if "neko_hip_create" in b)
    lines = [ln for ln in block.splitlines() if not ln.startswith("#include")]
    src = ("#include <stdio.h>\n#include <stdint.h>\n#include \"neko_hip.h\"\n"
           "void example(void* x, void* xn, const float* w, void* qkv, const int32_t* positions, const float* wqk,\n"
           "             const float* cs, void* h, void* g, uint16_t* k_cache, uint16_t* v_cache, void* delta,\n"
           "             const uint8_t* w_gate_up, float* gu, void* att) {\n" + "\n".join(lines) + "\n}\n")
    _compile(tmp_path, "example.c", src, "gcc", ["-std=c11", "-Wall", "-Werror", "-Wno-unused-variable",
                                                 "-I", os.path.join(ROOT, "include")])
