// HipBackend: neko::gpu::ComputeBackend over the neko_hip C ABI (replaces VulkanBackend /
// GlesBackend for the per-row ops; reference vk_compute.cpp, gl_compute.cpp).
//
// One C-ABI context = one in-order HIP stream, so dispatches are ordered without the barrier the
// Vulkan backend records after every dispatch (vk_compute.cpp:149-180). begin() and flush() have
// nothing to do: work is submitted as it is dispatched. The reference's shaders rely on robust
// buffer access for out-of-range indices; here every dispatch is checked against the bound buffer
// sizes before launch and an out-of-range request throws instead.
#include <algorithm>
#include <cstring>
#include <vector>

#include "../../include/neko_hip.h"
#include "compute.h"

namespace neko::gpu {
namespace {

struct HipBuffer : Buffer {
    void* dev = nullptr;
};

const char* kernelName(Kernel k) {
    static const char* const names[] = {"Embed",    "LayerNorm", "Matmul",   "KvStore",      "Attention", "Rope",
                                        "SiluMul",  "MatmulQ8",  "MatmulQ4", "GatedRmsNorm", "Gelu",      "AddRmsNorm"};
    const int i = static_cast<int>(k);
    return i >= 0 && i < static_cast<int>(Kernel::Count) ? names[i] : "?";
}

class HipBackend final : public ComputeBackend {
public:
    HipBackend() {
        if (neko_hip_create(0, &ctx_) != NEKO_OK) fail(std::string("HIP: ") + neko_hip_last_error(nullptr));
    }

    ~HipBackend() override {
        for (auto& b : buffers_) neko_hip_free(ctx_, b->dev);
        neko_hip_destroy(ctx_);
    }

    const char* name() const override { return "HIP"; }

    std::string deviceName() const override {
        char buf[256];
        neko_hip_device_name(ctx_, buf, sizeof buf);
        return buf;
    }

    size_t maxBufferBytes() const override { return neko_hip_max_buffer_bytes(ctx_); }

    Buffer* create(size_t bytes, const void* init, bool /*readback*/) override {
        auto b = std::make_unique<HipBuffer>();
        b->size = bytes;
        check(neko_hip_alloc(ctx_, bytes, &b->dev));
        buffers_.push_back(std::move(b));
        HipBuffer* hb = buffers_.back().get();
        if (init) check(neko_hip_upload(ctx_, hb->dev, init, bytes));
        else check(neko_hip_memset(ctx_, hb->dev, 0, bytes));
        return hb;
    }

    void upload(Buffer* b, size_t offset, const void* src, size_t bytes) override {
        HipBuffer* hb = as(b, "upload");
        if (offset > hb->size || bytes > hb->size - offset) fail("HIP upload: range outside the buffer");
        check(neko_hip_upload(ctx_, static_cast<char*>(hb->dev) + offset, src, bytes));
    }

    void download(Buffer* b, size_t offset, void* dst, size_t bytes) override {
        HipBuffer* hb = as(b, "download");
        if (offset > hb->size || bytes > hb->size - offset) fail("HIP download: range outside the buffer");
        check(neko_hip_download(ctx_, dst, static_cast<char*>(hb->dev) + offset, bytes));
    }

    void begin() override {}
    void flush() override {}
    void submitAndWait() override { check(neko_hip_synchronize(ctx_)); }

    void dispatch(Kernel k, Buffer* const bindings[4], const int32_t params[8], uint32_t gx, uint32_t gy) override {
        const int32_t* pa = params;
        const int32_t* pb = params + 4;
        switch (k) {
            case Kernel::Embed: embed(bindings, pa, pb); return;
            case Kernel::LayerNorm: layerNorm(bindings, pa, gx); return;
            case Kernel::Rope: rope(bindings, pa, pb, gx, gy); return;
            case Kernel::SiluMul: siluMul(bindings, pa); return;
            case Kernel::GatedRmsNorm: gatedRmsNorm(bindings, pa, gx); return;
            case Kernel::Gelu: gelu(bindings, pa); return;
            case Kernel::KvStore: kvStore(bindings, pa, pb); return;
            case Kernel::AddRmsNorm: addRmsNorm(bindings, pa, gx); return;
            case Kernel::Attention: attention(bindings, pa, pb); return;
            case Kernel::Matmul: matmul(bindings, pa, pb, gx, NEKO_FMT_F16); return;
            case Kernel::MatmulQ8: matmul(bindings, pa, pb, gx, NEKO_FMT_FP8); return;
            case Kernel::MatmulQ4: matmul(bindings, pa, pb, gx, NEKO_FMT_FP4); return;
            default: break;
        }
        fail(std::string("HIP backend: unknown kernel ") + kernelName(k));
    }

private:
    void check(int rc) const {
        if (rc != NEKO_OK) fail(std::string("HIP: ") + neko_hip_last_error(ctx_));
    }

    static HipBuffer* as(Buffer* b, const char* what) {
        auto* hb = dynamic_cast<HipBuffer*>(b);
        if (!hb) fail(std::string("HIP ") + what + ": missing or foreign buffer");
        return hb;
    }

    // Binding i must hold at least `bytes` bytes.
    static void* need(Buffer* const bindings[4], int i, uint64_t bytes, const char* what) {
        HipBuffer* b = as(bindings[i], what);
        if (bytes > b->size)
            fail(std::string("HIP ") + what + ": binding " + std::to_string(i) + " holds " + std::to_string(b->size) +
                 " bytes, the dispatch reads " + std::to_string(bytes));
        return b->dev;
    }

    // Byte counts for the bounds checks, failing rather than wrapping (grid sizes are 32-bit and the
    // parameters 31-bit, so their products can pass 64 bits).
    static uint64_t mul(uint64_t a, uint64_t b, uint64_t c = 1) {
        uint64_t ab = 0, abc = 0;
        if (__builtin_mul_overflow(a, b, &ab) || __builtin_mul_overflow(ab, c, &abc))
            fail("HIP: dispatch size overflows 64 bits");
        return abc;
    }
    static uint64_t add(uint64_t a, uint64_t b) {
        uint64_t r = 0;
        if (__builtin_add_overflow(a, b, &r)) fail("HIP: dispatch size overflows 64 bits");
        return r;
    }

    static void positive(int64_t v, const char* what) {
        if (v < 0) fail(std::string("HIP ") + what + ": negative parameter");
    }

    void embed(Buffer* const b[4], const int32_t* pa, const int32_t* pb) {
        const int64_t T = pa[0], C = pa[1], pos0 = pa[2];
        const int flags = pa[3];
        const int64_t rowBase = pb[0], rows = pb[1], rowWords = pb[2];
        positive(T, "Embed");
        positive(C, "Embed");
        positive(rows, "Embed");
        if (T == 0 || C == 0 || rows == 0) return;
        const int fmt = (flags & 2) ? NEKO_FMT_FP8 : (flags & 4) ? NEKO_FMT_FP4 : NEKO_FMT_F16;
        // The F16 table is indexed row * C halves; quantized tables by row * rowWords words (embed.comp:23-36).
        const int64_t rowBytes = fmt == NEKO_FMT_F16 ? 2 * C : 4 * rowWords;
        void* tokens = need(b, 0, mul(T, 4), "Embed");
        void* table = need(b, 1, mul(rows, rowBytes), "Embed");
        void* out = need(b, 3, mul(T, C, 4), "Embed");
        if (flags & 8) {
            // Granite's embedding multiplier (granite_model.cpp:298-301), its bits in PB[3].
            if (flags & 1) fail("HIP Embed: a position table and a multiplier are not combined");
            check(neko_hip_embed_scaled(ctx_, static_cast<const int32_t*>(tokens), T, table, rowBytes, fmt, C, rowBase,
                                        rows, bitsFloat(pb[3]), out, C, NEKO_DT_F32));
            return;
        }
        const uint16_t* wpe = nullptr;
        int64_t wpeRows = 0;
        if (flags & 1) {
            HipBuffer* w = as(b[2], "Embed");
            wpe = static_cast<const uint16_t*>(w->dev);
            wpeRows = int64_t(w->size / (uint64_t(C) * 2));
        }
        check(neko_hip_embed(ctx_, static_cast<const int32_t*>(tokens), T, table, rowBytes, fmt, C, rowBase, rows, wpe,
                             wpeRows, pos0, out, C, NEKO_DT_F32));
    }

    void layerNorm(Buffer* const b[4], const int32_t* pa, uint32_t gx) {
        const int64_t C = pa[0], rowOffset = pa[2], rows = gx;
        const float eps = bitsFloat(pa[1]);
        const bool rms = (pa[3] & 1) != 0;
        positive(C, "LayerNorm");
        positive(rowOffset, "LayerNorm");
        if (rows == 0 || C == 0) return;
        auto* x = static_cast<const float*>(need(b, 0, mul(rowOffset + rows, C, 4), "LayerNorm"));
        void* y = need(b, 1, mul(rows, C, 4), "LayerNorm");
        auto* g = static_cast<const float*>(need(b, 2, mul(C, 4), "LayerNorm"));
        if (rms) {
            check(neko_hip_rmsnorm(ctx_, x + rowOffset * C, C, y, C, g, rows, C, eps, NEKO_DT_F32));
        } else {
            auto* beta = static_cast<const float*>(need(b, 3, mul(C, 4), "LayerNorm"));
            check(neko_hip_layernorm(ctx_, x + rowOffset * C, C, y, C, g, beta, rows, C, eps, NEKO_DT_F32));
        }
    }

    void rope(Buffer* const b[4], const int32_t* pa, const int32_t* pb, uint32_t gx, uint32_t gy) {
        const int64_t stride = pa[0], nHead = pa[1], hd = pa[2], pos0 = pa[3], T = gy;
        const int64_t nKv = int64_t(gx) - nHead;
        const float eps = bitsFloat(pb[0]);
        const bool norm = (pb[1] & 1) != 0;
        positive(nHead, "Rope");
        positive(nKv, "Rope");
        positive(pos0, "Rope");
        if (hd <= 0 || hd % 2 != 0 || hd > 512) fail("HIP Rope: head dim must be even and <= 512");
        if (T == 0 || gx == 0) return;
        if (stride < int64_t(gx) * hd) fail("HIP Rope: qkv stride shorter than the heads it covers");
        void* qkv = need(b, 0, mul(add(mul(T - 1, stride), mul(gx, hd)), 4), "Rope");
        const float* wn = norm ? static_cast<const float*>(need(b, 1, uint64_t(2 * hd) * 4, "Rope")) : nullptr;
        HipBuffer* cs = as(b[2], "Rope");
        const int64_t nPos = int64_t(cs->size / (uint64_t(hd) * 4));
        if (pos0 + T > nPos) fail("HIP Rope: positions run past the cos/sin table");
        check(neko_hip_qk_norm_rope(ctx_, qkv, stride, T, int(nHead), int(nKv), int(hd), pos0, nullptr, wn,
                                    static_cast<const float*>(cs->dev), nPos, eps, NEKO_DT_F32));
    }

    void siluMul(Buffer* const b[4], const int32_t* pa) {
        const int64_t T = pa[0], I = pa[1];
        positive(T, "SiluMul");
        positive(I, "SiluMul");
        if (T == 0 || I == 0) return;
        void* h = need(b, 0, mul(T, 2 * I, 4), "SiluMul");
        void* g = need(b, 1, mul(T, I, 4), "SiluMul");
        check(neko_hip_swiglu(ctx_, h, 2 * I, g, I, T, I, NEKO_DT_F32));
    }

    void gatedRmsNorm(Buffer* const b[4], const int32_t* pa, uint32_t gx) {
        const int64_t D = pa[0], groups = pa[2], zStride = pa[3], rows = gx;
        const float eps = bitsFloat(pa[1]);
        positive(D, "GatedRmsNorm");
        if (groups <= 0 || D % groups != 0) fail("HIP GatedRmsNorm: groups must divide D");
        if (zStride < D) fail("HIP GatedRmsNorm: z stride shorter than D");
        if (rows == 0 || D == 0) return;
        void* y = need(b, 0, mul(rows, D, 4), "GatedRmsNorm");
        void* z = need(b, 1, mul(add(mul(rows - 1, zStride), D), 4), "GatedRmsNorm");
        auto* w = static_cast<const float*>(need(b, 2, mul(D, 4), "GatedRmsNorm"));
        check(neko_hip_gated_rmsnorm(ctx_, y, D, z, zStride, y, D, w, rows, D, int(groups), eps, NEKO_DT_F32));
    }

    void gelu(Buffer* const b[4], const int32_t* pa) {
        const int64_t n = pa[0];
        positive(n, "Gelu");
        if (n == 0) return;
        void* x = need(b, 0, mul(n, 4), "Gelu");
        void* y = need(b, 1, mul(n, 4), "Gelu");
        check(neko_hip_gelu_tanh(ctx_, x, y, n, NEKO_DT_F32));
    }

    // kv_store.comp: PA (T, width, pos0), PB (rowStride, kOffset, vOffset); caches [ctx][width] f16.
    void kvStore(Buffer* const b[4], const int32_t* pa, const int32_t* pb) {
        const int64_t T = pa[0], W = pa[1], pos0 = pa[2], stride = pb[0], kOff = pb[1], vOff = pb[2];
        positive(T, "KvStore");
        positive(W, "KvStore");
        positive(pos0, "KvStore");
        positive(kOff, "KvStore");
        positive(vOff, "KvStore");
        if (T == 0 || W == 0) return;
        if (stride < kOff + W || stride < vOff + W) fail("HIP KvStore: k/v columns exceed the qkv row stride");
        void* qkv = need(b, 0, mul(add(mul(T - 1, stride), std::max(kOff, vOff) + W), 4), "KvStore");
        auto* kc = static_cast<uint16_t*>(need(b, 1, mul(pos0 + T, W, 2), "KvStore"));
        auto* vc = static_cast<uint16_t*>(need(b, 2, mul(pos0 + T, W, 2), "KvStore"));
        check(neko_hip_store_kv(ctx_, qkv, stride, kOff, vOff, T, W, pos0, nullptr, kc, vc, pos0 + T, NEKO_DT_F32));
    }

    // attention.comp: PA (T, qStride, nHead, pos0), PB (headDim, scale bits, kvWidth); bindings qkv
    // (f32 rows of qStride, head h of token t at t*qStride + h*hd), the k and v caches (f16 rows of
    // kvWidth, positions 0 .. pos0 + T - 1), out (f32 [T][nHead*hd]); dispatch (nHead, T).
    void attention(Buffer* const b[4], const int32_t* pa, const int32_t* pb) {
        const int64_t T = pa[0], qs = pa[1], H = pa[2], pos0 = pa[3], hd = pb[0], kvw = pb[2];
        const float scale = bitsFloat(pb[1]);
        positive(T, "Attention");
        positive(qs, "Attention");
        positive(pos0, "Attention");
        if (T == 0) return;
        if (H <= 0 || hd <= 0 || kvw <= 0 || kvw % hd || H % (kvw / hd))
            fail("HIP Attention: nHead must be a multiple of kvWidth / headDim");
        void* q = need(b, 0, mul(add(mul(T - 1, qs), mul(H, hd)), 4), "Attention");
        auto* kc = static_cast<const uint16_t*>(need(b, 1, mul(pos0 + T, kvw, 2), "Attention"));
        auto* vc = static_cast<const uint16_t*>(need(b, 2, mul(pos0 + T, kvw, 2), "Attention"));
        void* out = need(b, 3, mul(mul(T, H), hd, 4), "Attention");
        check(neko_hip_attention(ctx_, q, qs, kc, vc, out, H * hd, T, static_cast<int>(H), static_cast<int>(kvw / hd),
                                 static_cast<int>(hd), pos0, scale, NEKO_DT_F32));
    }

    // Residual add + RMSNorm: PA (C, eps); bindings x (in/out), delta, xn, w; dispatch (rows, 1).
    void addRmsNorm(Buffer* const b[4], const int32_t* pa, uint32_t gx) {
        const int64_t C = pa[0], rows = gx;
        const float eps = bitsFloat(pa[1]);
        positive(C, "AddRmsNorm");
        if (rows == 0 || C == 0) return;
        void* x = need(b, 0, mul(rows, C, 4), "AddRmsNorm");
        void* d = need(b, 1, mul(rows, C, 4), "AddRmsNorm");
        void* xn = need(b, 2, mul(rows, C, 4), "AddRmsNorm");
        auto* w = static_cast<const float*>(need(b, 3, mul(C, 4), "AddRmsNorm"));
        check(neko_hip_add_rmsnorm(ctx_, x, C, d, C, xn, C, w, rows, C, eps, NEKO_DT_F32));
    }

    // matmul.comp / matmul_q8.comp / matmul_q4.comp: PA (K, N = the row stride of y, T, flags: 1 GELU,
    // 2 accumulate, 4 bias), PB (xRow0, nOffset); bindings x rows of K, the weight rows, bias, y;
    // dispatch (weight rows, ceil(T / 4)). y[t][nOffset + n] (+)= act(x[xRow0 + t] . W[n] + bias[n]).
    void matmul(Buffer* const b[4], const int32_t* pa, const int32_t* pb, uint32_t gx, int fmt) {
        const int64_t K = pa[0], N = pa[1], T = pa[2], row0 = pb[0], nOff = pb[1], rows = gx;
        const int flags = pa[3];
        const char* what = fmt == NEKO_FMT_F16 ? "Matmul" : fmt == NEKO_FMT_FP8 ? "MatmulQ8" : "MatmulQ4";
        positive(K, what);
        positive(N, what);
        positive(T, what);
        positive(row0, what);
        positive(nOff, what);
        if (T == 0 || rows == 0) return;
        if (nOff + rows > N) fail(std::string("HIP ") + what + ": output columns exceed the row stride of y");
        const uint64_t rb = neko_quant_row_bytes(fmt, K);
        auto* x = static_cast<char*>(need(b, 0, mul(row0 + T, K, 4), what)) + row0 * K * 4;
        void* w = need(b, 1, mul(rows, rb), what);
        const float* bias = (flags & 4) ? static_cast<const float*>(need(b, 2, mul(rows, 4), what)) : nullptr;
        auto* y = static_cast<char*>(need(b, 3, mul(add(mul(T - 1, N), nOff + rows), 4), what)) + nOff * 4;
        check(neko_hip_matmul(ctx_, x, K, T, K, w, int64_t(rb), fmt, rows, bias, y, N, flags & 3, NEKO_DT_F32,
                              NEKO_DT_F32));
    }

    neko_hip_ctx* ctx_ = nullptr;
    std::vector<std::unique_ptr<HipBuffer>> buffers_;
};

}  // namespace

std::unique_ptr<ComputeBackend> createHip(std::string& error) {
    try {
        return std::make_unique<HipBackend>();
    } catch (const std::exception& e) {
        error = e.what();
        return nullptr;
    }
}

}  // namespace neko::gpu
