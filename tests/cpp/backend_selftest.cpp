// Port of the reference's GPU backend self-test (gpu/compute.cpp:32-290), every case, driven through
// neko::gpu::ComputeBackend::dispatch with the reference's own parameter blocks. The CPU side is the
// oracle (oracle/neko_oracle.c), standing where the reference calls its cpu:: ops. Same inputs scheme
// (std::mt19937(1234), uniform(-1, 1), f16-rounded weights), same shapes and the reference's tolerance
// test |gpu - cpu| <= tol * (1 + |cpu|); the gather cases additionally require bit equality.
//
// Built into tests/cpp/_build/libbackend_selftest.so and called from tests/test_gpu_backend.py.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../nekochat_amd/csrc/compute.h"
#include "../../oracle/neko_oracle.h"

using namespace neko;
using namespace neko::gpu;

namespace {

struct Failure {
    std::string msg;
};

void closeOrFail(const std::vector<float>& gpu, const std::vector<float>& cpu, float tol, const char* what, bool exact) {
    for (size_t i = 0; i < gpu.size(); i++) {
        const float d = std::fabs(gpu[i] - cpu[i]);
        const bool bitsEqual = std::memcmp(&gpu[i], &cpu[i], 4) == 0;
        if (!(d <= tol * (1.0f + std::fabs(cpu[i]))) || (exact && !bitsEqual)) {
            char buf[256];
            std::snprintf(buf, sizeof buf, "self-test %s mismatch at %zu: gpu %.9g cpu %.9g%s", what, i, gpu[i], cpu[i],
                          exact ? " (bit-exact required)" : "");
            throw Failure{buf};
        }
    }
}

struct Harness {
    ComputeBackend& be;
    std::mt19937 rng{1234};
    std::uniform_real_distribution<float> u{-1.0f, 1.0f};

    std::vector<float> rnd(size_t n) {
        std::vector<float> v(n);
        for (auto& x : v) x = u(rng);
        return v;
    }
    // Rounds v to f16 in place and returns the bits.
    static std::vector<uint16_t> halves(std::vector<float>& v) {
        std::vector<uint16_t> h(v.size());
        for (size_t i = 0; i < v.size(); i++) {
            h[i] = oracle_f32_to_f16(v[i]);
            v[i] = oracle_f16_to_f32(h[i]);
        }
        return h;
    }
    void run(Kernel k, std::initializer_list<Buffer*> b, std::initializer_list<int32_t> p, uint32_t gx, uint32_t gy) {
        Buffer* binds[4] = {};
        int32_t params[8] = {};
        std::copy(b.begin(), b.end(), binds);
        std::copy(p.begin(), p.end(), params);
        be.dispatch(k, binds, params, gx, gy);
    }
    std::vector<float> read(Buffer* b, size_t n) {
        std::vector<float> v(n);
        be.download(b, 0, v.data(), n * 4);
        return v;
    }

    void embed() {  // compute.cpp:106-132
        const int EV = 10, EC = 64, EP = 4, ET = 3, epos = 1, split = 6;
        auto wte = rnd(size_t(EV * EC)), wpe = rnd(size_t(EP * EC));
        auto hte = halves(wte), hpe = halves(wpe);
        int32_t toks[ET] = {3, 7, 9};
        std::vector<float> ref(size_t(ET * EC)), refNoPos(size_t(ET * EC));
        for (int t = 0; t < ET; t++)
            for (int c = 0; c < EC; c++) {
                refNoPos[size_t(t * EC + c)] = wte[size_t(toks[t] * EC + c)];
                ref[size_t(t * EC + c)] = wte[size_t(toks[t] * EC + c)] + wpe[size_t((epos + t) * EC + c)];
            }
        Buffer* bt = be.create(sizeof toks, toks);
        Buffer* out = be.create(ref.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::Embed, {bt, be.create(hte.size() * 2, hte.data()), be.create(hpe.size() * 2, hpe.data()), out},
            {ET, EC, epos, 1, 0, EV}, 1, ET);
        be.submitAndWait();
        closeOrFail(read(out, ref.size()), ref, 1e-5f, "embed", true);
        Buffer* c0 = be.create(size_t(split * EC) * 2, hte.data());
        Buffer* c1 = be.create(size_t((EV - split) * EC) * 2, hte.data() + split * EC);
        be.begin();
        run(Kernel::Embed, {bt, c0, nullptr, out}, {ET, EC, 0, 0, 0, split}, 1, ET);
        run(Kernel::Embed, {bt, c1, nullptr, out}, {ET, EC, 0, 0, split, EV - split}, 1, ET);
        be.submitAndWait();
        closeOrFail(read(out, ref.size()), refNoPos, 1e-5f, "embed-chunked", true);
    }

    void norms() {  // compute.cpp:134-154
        const int C = 96, R = 3;
        auto lx = rnd(size_t(C * R)), g = rnd(size_t(C)), b = rnd(size_t(C));
        for (auto& v : lx) v *= 20.0f;
        std::vector<float> lref(lx.size()), rref(lx.size());
        oracle_layernorm(lx.data(), lref.data(), g.data(), b.data(), R, C, 1e-5f);
        oracle_rmsnorm(lx.data(), rref.data(), g.data(), R, C, 1e-6f);
        Buffer* blx = be.create(lx.size() * 4, lx.data());
        Buffer* bg = be.create(g.size() * 4, g.data());
        Buffer* bbb = be.create(b.size() * 4, b.data());
        Buffer* bly = be.create(lx.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::LayerNorm, {blx, bly, bg, bbb}, {C, floatBits(1e-5f), 0, 0}, R, 1);
        be.submitAndWait();
        closeOrFail(read(bly, lx.size()), lref, 1e-3f, "layernorm", false);
        be.begin();
        run(Kernel::LayerNorm, {blx, bly, bg, nullptr}, {C, floatBits(1e-6f), 0, 1}, R, 1);
        be.submitAndWait();
        closeOrFail(read(bly, lx.size()), rref, 1e-3f, "rmsnorm", false);
        // rowOffset: the final-norm form, one row normalised from row R - 1 (gpt2_model.cpp:274).
        Buffer* one = be.create(size_t(C) * 4, nullptr, true);
        be.begin();
        run(Kernel::LayerNorm, {blx, one, bg, bbb}, {C, floatBits(1e-5f), R - 1, 0}, 1, 1);
        be.submitAndWait();
        std::vector<float> last(lref.end() - C, lref.end());
        closeOrFail(read(one, size_t(C)), last, 1e-3f, "layernorm-rowOffset", false);
        // Chained dispatches in one submission (layernorm -> gelu reading its output, compute.cpp:156-176).
        Buffer* bgl = be.create(lx.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::LayerNorm, {blx, bly, bg, bbb}, {C, floatBits(1e-5f), 0, 0}, R, 1);
        run(Kernel::Gelu, {bly, bgl}, {C * R}, uint32_t((C * R + 63) / 64), 1);
        be.submitAndWait();
        std::vector<float> gref(lref.size());
        for (size_t i = 0; i < gref.size(); i++) gref[i] = oracle_gelu(lref[i]);
        closeOrFail(read(bgl, gref.size()), gref, 1e-3f, "chained layernorm->gelu", false);
    }

    void rope() {  // compute.cpp:178-202
        const int H = 2, KV = 1, hd = 64, T = 2, pos0 = 3, stride = (H + 2 * KV) * hd;
        auto qkv = rnd(size_t(T * stride)), wn = rnd(size_t(2 * hd));
        std::vector<float> cs(size_t((pos0 + T) * hd));
        for (int p = 0; p < pos0 + T; p++)
            for (int i = 0; i < hd / 2; i++) {
                double a = p * std::pow(10000.0, -2.0 * i / hd);
                cs[size_t(p * hd + 2 * i)] = float(std::cos(a));
                cs[size_t(p * hd + 2 * i + 1)] = float(std::sin(a));
            }
        std::vector<float> ref = qkv;
        for (int t = 0; t < T; t++) {
            float* r = ref.data() + t * stride;
            oracle_rmsnorm(r, r, wn.data(), H, hd, 1e-6f);
            oracle_rmsnorm(r + H * hd, r + H * hd, wn.data() + hd, KV, hd, 1e-6f);
            oracle_rope(r, H + KV, hd, cs.data() + (pos0 + t) * hd);
        }
        Buffer* bq = be.create(qkv.size() * 4, qkv.data(), true);
        be.begin();
        run(Kernel::Rope, {bq, be.create(wn.size() * 4, wn.data()), be.create(cs.size() * 4, cs.data())},
            {stride, H, hd, pos0, floatBits(1e-6f), 1}, H + KV, T);
        be.submitAndWait();
        closeOrFail(read(bq, ref.size()), ref, 1e-3f, "rope", false);
    }

    void siluMul() {  // compute.cpp:204-216
        const int T = 2, I = 100;
        auto h = rnd(size_t(T * 2 * I));
        for (auto& v : h) v *= 6.0f;
        std::vector<float> ref(size_t(T * I));
        oracle_silu_mul(h.data(), ref.data(), T, I);
        Buffer* bo = be.create(ref.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::SiluMul, {be.create(h.size() * 4, h.data()), bo}, {T, I}, uint32_t((I + 63) / 64), T);
        be.submitAndWait();
        closeOrFail(read(bo, ref.size()), ref, 1e-4f, "silu_mul", false);
    }

    void quantEmbed() {  // compute.cpp:245-260
        for (int fmt : {ORACLE_FMT_FP8, ORACLE_FMT_FP4}) {
            const int EV = 10, EC = 64, ET = 3;
            auto table = rnd(size_t(EV * EC));
            const size_t rb = oracle_quant_row_bytes(fmt, EC);
            std::vector<uint8_t> q(rb * EV);
            oracle_quantize_rows(fmt, EV, EC, table.data(), q.data());
            int32_t toks[ET] = {3, 7, 9};
            std::vector<float> ref(size_t(ET * EC));
            for (int t = 0; t < ET; t++) oracle_dequantize_row(fmt, EC, q.data() + rb * size_t(toks[t]), ref.data() + t * EC);
            Buffer* out = be.create(ref.size() * 4, nullptr, true);
            be.begin();
            run(Kernel::Embed, {be.create(sizeof toks, toks), be.create(q.size(), q.data()), nullptr, out},
                {ET, EC, 0, fmt == ORACLE_FMT_FP8 ? 2 : 4, 0, EV, int(rb / 4)}, 1, ET);
            be.submitAndWait();
            closeOrFail(read(out, ref.size()), ref, 1e-5f, fmt == ORACLE_FMT_FP8 ? "embed-FP8" : "embed-FP4", true);
        }
    }

    void scaledEmbed() {  // granite_model.cpp:298-301 through Embed flag 8 (the multiplier's bits in PB[3])
        for (int fmt : {ORACLE_FMT_F16, ORACLE_FMT_FP8, ORACLE_FMT_FP4}) {
            const int EV = 10, EC = 64, ET = 3;
            const float mult = 12.0f;  // Granite-4.0's embedding_multiplier
            auto table = rnd(size_t(EV * EC));
            const size_t rb = oracle_quant_row_bytes(fmt, EC);
            std::vector<uint8_t> q(rb * EV);
            oracle_quantize_rows(fmt, EV, EC, table.data(), q.data());
            int32_t toks[ET] = {3, 7, 9};
            std::vector<float> ref(size_t(ET * EC));
            for (int t = 0; t < ET; t++) {
                oracle_dequantize_row(fmt, EC, q.data() + rb * size_t(toks[t]), ref.data() + t * EC);
                for (int c = 0; c < EC; c++) ref[size_t(t * EC + c)] *= mult;  // x[c] *= embeddingMult
            }
            Buffer* out = be.create(ref.size() * 4, nullptr, true);
            const int32_t ff = fmt == ORACLE_FMT_FP8 ? 2 : fmt == ORACLE_FMT_FP4 ? 4 : 0;
            be.begin();
            run(Kernel::Embed, {be.create(sizeof toks, toks), be.create(q.size(), q.data()), nullptr, out},
                {ET, EC, 0, ff | 8, 0, EV, fmt == ORACLE_FMT_F16 ? EC / 2 : int(rb / 4), floatBits(mult)}, 1, ET);
            be.submitAndWait();
            closeOrFail(read(out, ref.size()), ref, 0.0f, "embed scaled", true);
        }
    }

    void gatedNorm() {  // granite_model.cpp:278-287 through the GatedRmsNorm extension
        const int T = 3, D = 128, groups = 2, zStride = 200;
        auto y = rnd(size_t(T * D)), z = rnd(size_t(T * zStride)), w = rnd(size_t(D));
        for (auto& v : z) v *= 4.0f;
        std::vector<float> ref = y;
        oracle_gated_rmsnorm(ref.data(), z.data(), zStride, w.data(), T, D, groups, 1e-5f);
        Buffer* by = be.create(y.size() * 4, y.data(), true);
        be.begin();
        run(Kernel::GatedRmsNorm, {by, be.create(z.size() * 4, z.data()), be.create(w.size() * 4, w.data())},
            {D, floatBits(1e-5f), groups, zStride}, T, 1);
        be.submitAndWait();
        closeOrFail(read(by, ref.size()), ref, 1e-3f, "gated-rmsnorm", false);
    }

    void kvStore() {  // kv_store.comp / cpu::storeKv through the reference's KvStore parameter blocks
        const int T = 3, KW = 64, QH = 128, QW = QH + 2 * KW, pos0 = 2, ctx = 8;
        auto qkv = rnd(size_t(T * QW));
        for (auto& v : qkv) v *= 3.0f;
        std::vector<uint16_t> kref(size_t(ctx * KW), 0), vref(kref);
        oracle_store_kv(qkv.data() + QH, qkv.data() + QH + KW, QW, kref.data(), vref.data(), KW, T, pos0);
        std::vector<uint16_t> zero(kref.size(), 0);
        Buffer* bk = be.create(zero.size() * 2, zero.data(), true);
        Buffer* bv = be.create(zero.size() * 2, zero.data(), true);
        be.begin();
        run(Kernel::KvStore, {be.create(qkv.size() * 4, qkv.data()), bk, bv}, {T, KW, pos0, 0, QW, QH, QH + KW},
            uint32_t((KW / 2 + 63) / 64), T);
        be.submitAndWait();
        std::vector<uint16_t> k(kref.size()), v(vref.size());
        be.download(bk, 0, k.data(), k.size() * 2);
        be.download(bv, 0, v.data(), v.size() * 2);
        if (k != kref || v != vref) throw Failure{"self-test kv-store mismatch (bit-exact required)"};
    }

    void addRmsNorm() {  // the residual add of a kAccumulate matmul epilogue + RMSNorm, AddRmsNorm extension
        const int T = 4, C = 96;
        auto x = rnd(size_t(T * C)), d = rnd(size_t(T * C)), w = rnd(size_t(C));
        halves(w);
        std::vector<float> xr = x, xn(x.size());
        oracle_add_rmsnorm(xr.data(), d.data(), xn.data(), w.data(), T, C, 1e-6f);
        Buffer* bx = be.create(x.size() * 4, x.data(), true);
        Buffer* bn = be.create(x.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::AddRmsNorm, {bx, be.create(d.size() * 4, d.data()), bn, be.create(w.size() * 4, w.data())},
            {C, floatBits(1e-6f)}, T, 1);
        be.submitAndWait();
        closeOrFail(read(bx, xr.size()), xr, 0.0f, "add-rmsnorm residual", true);
        closeOrFail(read(bn, xn.size()), xn, 1e-3f, "add-rmsnorm", false);
    }

    // y[t][nOff + n] = y0 + oracle matmul (bias, no accumulate), the reference cases' expected value.
    static std::vector<float> expected(int fmt, const std::vector<float>& x, int T, int K, const std::vector<uint8_t>& w,
                                       int N, const std::vector<float>& bias, int flags, const std::vector<float>& y0,
                                       int NS, int nOff) {
        std::vector<float> v(size_t(T) * size_t(N), 0.0f), ref = y0;
        oracle_matmul(fmt, x.data(), T, K, w.data(), int64_t(w.size() / size_t(N)), N, bias.data(), v.data(), flags & 1);
        for (int t = 0; t < T; t++)
            for (int n = 0; n < N; n++) {
                float& dst = ref[size_t(t * NS + nOff + n)];
                dst = (flags & 2) ? dst + v[size_t(t * N + n)] : v[size_t(t * N + n)];
            }
        return ref;
    }

    void matmul() {  // compute.cpp:63-104 (F16 rows) and 208-244 (FP8 / FP4 rows)
        {   // bias + GELU, T = 5 (a partial 4-token tile)
            const int K = 64, N = 37, T = 5;
            auto x = rnd(size_t(T * K)), bias = rnd(size_t(N)), wf = rnd(size_t(N * K));
            auto w = halves(wf);
            std::vector<uint8_t> wb(w.size() * 2);
            std::memcpy(wb.data(), w.data(), wb.size());
            const auto ref = expected(ORACLE_FMT_F16, x, T, K, wb, N, bias, 1, std::vector<float>(size_t(T * N)), N, 0);
            Buffer* by = be.create(ref.size() * 4, nullptr, true);
            be.begin();
            run(Kernel::Matmul, {be.create(x.size() * 4, x.data()), be.create(wb.size(), wb.data()),
                                 be.create(bias.size() * 4, bias.data()), by},
                {K, N, T, 4 | 1}, uint32_t(N), uint32_t((T + 3) / 4));
            be.submitAndWait();
            closeOrFail(read(by, ref.size()), ref, 2e-3f, "matmul", false);
        }
        {   // K = 768, x row offset, accumulate, output column offset
            const int BK = 768, BN = 96, BT = 6, row0 = 1, nOff = 5, NS = BN + 8;
            auto bx = rnd(size_t((BT + row0) * BK)), bb = rnd(size_t(BN)), bwf = rnd(size_t(BN * BK));
            auto y0 = rnd(size_t(BT * NS));
            auto bw = halves(bwf);
            std::vector<uint8_t> wb(bw.size() * 2);
            std::memcpy(wb.data(), bw.data(), wb.size());
            const std::vector<float> xs(bx.begin() + row0 * BK, bx.end());
            const auto ref = expected(ORACLE_FMT_F16, xs, BT, BK, wb, BN, bb, 2, y0, NS, nOff);
            Buffer* by = be.create(y0.size() * 4, y0.data(), true);
            be.begin();
            run(Kernel::Matmul, {be.create(bx.size() * 4, bx.data()), be.create(wb.size(), wb.data()),
                                 be.create(bb.size() * 4, bb.data()), by},
                {BK, NS, BT, 4 | 2, row0, nOff}, uint32_t(BN), uint32_t((BT + 3) / 4));
            be.submitAndWait();
            closeOrFail(read(by, ref.size()), ref, 2e-3f, "matmul-768", false);
        }
        // FP8 / FP4 rows: bias + accumulate + output offset, K = 96 and 1024, T = 5.
        for (int fmt : {ORACLE_FMT_FP8, ORACLE_FMT_FP4}) {
            for (int K : {96, 1024}) {
                const int N = 37, T = 5, nOff = 3, NS = N + 5;
                auto x = rnd(size_t(T * K)), bias = rnd(size_t(N)), wf = rnd(size_t(N * K)), y0 = rnd(size_t(T * NS));
                std::vector<uint8_t> wb(size_t(N) * oracle_quant_row_bytes(fmt, K));
                oracle_quantize_rows(fmt, N, K, wf.data(), wb.data());
                const auto ref = expected(fmt, x, T, K, wb, N, bias, 2, y0, NS, nOff);
                Buffer* by = be.create(y0.size() * 4, y0.data(), true);
                be.begin();
                run(fmt == ORACLE_FMT_FP8 ? Kernel::MatmulQ8 : Kernel::MatmulQ4,
                    {be.create(x.size() * 4, x.data()), be.create(wb.size(), wb.data()),
                     be.create(bias.size() * 4, bias.data()), by},
                    {K, NS, T, 4 | 2, 0, nOff}, uint32_t(N), uint32_t((T + 3) / 4));
                be.submitAndWait();
                closeOrFail(read(by, ref.size()), ref, 2e-3f, fmt == ORACLE_FMT_FP8 ? "FP8 matmul" : "FP4 matmul", false);
            }
        }
    }

    void attention() {  // compute.cpp:262-283: kv_store + grouped-query attention, pos0 > 1024
        const int H = 4, KV = 2, hd = 64, T = 3, pos0 = 1030, ctx = pos0 + T;
        const int stride = (H + 2 * KV) * hd, kvW = KV * hd, kOff = H * hd, vOff = (H + KV) * hd;
        auto qkv = rnd(size_t(T * stride));
        auto kf = rnd(size_t(ctx * kvW)), vf = rnd(size_t(ctx * kvW));
        auto kc = halves(kf), vc = halves(vf);
        std::vector<uint16_t> kcRef = kc, vcRef = vc;
        std::vector<float> ref(size_t(T * H * hd));
        oracle_store_kv(qkv.data() + kOff, qkv.data() + vOff, stride, kcRef.data(), vcRef.data(), kvW, T, pos0);
        oracle_attention(qkv.data(), stride, kcRef.data(), vcRef.data(), ref.data(), T, H, KV, hd, pos0);
        Buffer* bq = be.create(qkv.size() * 4, qkv.data());
        Buffer* bk = be.create(kc.size() * 2, kc.data());
        Buffer* bv = be.create(vc.size() * 2, vc.data());
        Buffer* bo = be.create(ref.size() * 4, nullptr, true);
        be.begin();
        run(Kernel::KvStore, {bq, bk, bv}, {T, kvW, pos0, 0, stride, kOff, vOff}, uint32_t((kvW / 2 + 63) / 64), T);
        run(Kernel::Attention, {bq, bk, bv, bo}, {T, stride, H, pos0, hd, floatBits(1.0f / std::sqrt(float(hd))), kvW},
            H, T);
        be.submitAndWait();
        closeOrFail(read(bo, ref.size()), ref, 2e-3f, "attention", false);
    }

    void unknownKernel() {  // a kernel id past the enum throws, not runs
        Buffer* b = be.create(64);
        try {
            run(Kernel::Count, {b, b, b, b}, {4, 4, 1, 0}, 4, 1);
        } catch (const NekoError&) {
            return;
        }
        throw Failure{"dispatch of an unknown kernel did not throw"};
    }

    void outOfRange() {  // a dispatch reading past a buffer throws instead of faulting
        Buffer* small = be.create(16);
        Buffer* g = be.create(96 * 4);
        bool threw = false;
        try {
            run(Kernel::LayerNorm, {small, small, g, g}, {96, floatBits(1e-5f), 0, 0}, 3, 1);
        } catch (const NekoError&) {
            threw = true;
        }
        if (!threw) throw Failure{"out-of-range LayerNorm dispatch did not throw"};
        threw = false;
        try {  // byte counts past 64 bits (2^32 - 1 rows of 2^31 - 1 floats) throw rather than wrap
            run(Kernel::LayerNorm, {small, small, g, g}, {0x7fffffff, floatBits(1e-5f), 1, 0}, 0xffffffffu, 1);
        } catch (const NekoError&) {
            threw = true;
        }
        if (!threw) throw Failure{"oversized LayerNorm dispatch did not throw"};
    }
};

}  // namespace

extern "C" int backend_selftest(char* err, int err_bytes) {
    std::string error;
    std::unique_ptr<ComputeBackend> be = createHip(error);
    if (!be) {
        std::snprintf(err, size_t(err_bytes), "createHip: %s", error.c_str());
        return 2;
    }
    try {
        Harness h{*be};
        h.embed();
        h.norms();
        h.rope();
        h.siluMul();
        h.quantEmbed();
        h.scaledEmbed();
        h.gatedNorm();
        h.kvStore();
        h.addRmsNorm();
        h.matmul();
        h.attention();
        h.unknownKernel();
        h.outOfRange();
        std::snprintf(err, size_t(err_bytes), "ok on %s (%s)", be->deviceName().c_str(), be->name());
        return 0;
    } catch (const Failure& f) {
        std::snprintf(err, size_t(err_bytes), "%s", f.msg.c_str());
    } catch (const std::exception& e) {
        std::snprintf(err, size_t(err_bytes), "self-test failed: %s", e.what());
    }
    return 1;
}

// createHip with no usable device returns null and an error string (factory convention) — runs on CPU.
extern "C" int backend_create_without_device(char* err, int err_bytes) {
    std::string error;
    std::unique_ptr<ComputeBackend> be = createHip(error);
    std::snprintf(err, size_t(err_bytes), "%s", error.c_str());
    return be ? 1 : 0;
}
