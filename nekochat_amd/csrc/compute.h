// The engine's per-op GPU backend contract, kept as the reference declares it so a HIP backend drops
// in beside its Vulkan and GLES backends (reference: shared/cpp/gpu/compute.h:14-58, common.h:26-31).
// Names, argument meaning, the Kernel numbering and the throw-on-failure convention are unchanged;
// GatedRmsNorm, Gelu and AddRmsNorm extend the enum after MatmulQ4, so existing values keep their
// numbers.
//
// Per-kernel parameter blocks (PA = params[0..3], PB = params[4..7]; floats travel as raw bits, see
// floatBits), activations f32, exactly as the reference's shaders take them:
//   Embed      PA (T, C, pos0, flags{1: + f16 wpe, 2: FP8 table, 4: FP4 table, 8: x *= PB[3]})
//              PB (rowBase, rows, rowWords = rowBytes / 4, multiplier bits for flag 8: Granite's
//              embedding_multiplier, granite_model.cpp:298-301)       bindings tokens, table, wpe, x
//   LayerNorm  PA (C, eps, rowOffset, flags{1: RMSNorm})     bindings x, y, gamma, beta; dispatch (rows, 1)
//   Rope       PA (qkvStride, nHead, headDim, pos0)
//              PB (eps, flags{1: per-head RMSNorm})           bindings qkv, wn[2 hd], cs; dispatch (nHead + nKv, T)
//   SiluMul    PA (T, I)                                     bindings h [T][2I], g [T][I]
//   GatedRmsNorm PA (D, eps, groups, zStride)                bindings y (in/out), z, w; dispatch (rows, 1)
//   Gelu       PA (n)                                        bindings x, y
//   KvStore    PA (T, width, pos0), PB (rowStride, kOffset, vOffset)   bindings qkv, kCache, vCache
//              (caches [ctx][width] f16)
//   AddRmsNorm PA (C, eps)                                   bindings x (in/out), delta, xn, w; dispatch (rows, 1)
//   Matmul / MatmulQ8 / MatmulQ4  PA (K, N = row stride of y, T, flags{1: GELU, 2: accumulate, 4: bias})
//              PB (xRow0, nOffset)                            bindings x, W rows (F16 / FP8 / FP4), bias, y;
//              dispatch (weight rows, ceil(T / 4))
// Attention is not implemented by the HIP backend: dispatching it throws NekoError.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

namespace neko {

struct NekoError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] inline void fail(const std::string& msg) { throw NekoError(msg); }

}  // namespace neko

namespace neko::gpu {

enum class Kernel : int {
    Embed = 0,
    LayerNorm,
    Matmul,
    KvStore,
    Attention,
    Rope,
    SiluMul,
    MatmulQ8,
    MatmulQ4,
    GatedRmsNorm,
    Gelu,
    AddRmsNorm,
    Count
};

struct Buffer {
    size_t size = 0;
    virtual ~Buffer() = default;
};

class ComputeBackend {
public:
    virtual ~ComputeBackend() = default;

    virtual const char* name() const = 0;
    virtual std::string deviceName() const = 0;
    virtual size_t maxBufferBytes() const = 0;

    // Buffers are owned by the backend and live until it is destroyed.
    virtual Buffer* create(size_t bytes, const void* init = nullptr, bool readback = false) = 0;
    virtual void upload(Buffer* b, size_t offset, const void* src, size_t bytes) = 0;
    virtual void download(Buffer* b, size_t offset, void* dst, size_t bytes) = 0;

    // begin(), any number of dispatch() (each ordered after the previous), submitAndWait().
    virtual void begin() = 0;
    virtual void dispatch(Kernel k, Buffer* const bindings[4], const int32_t params[8], uint32_t gx, uint32_t gy) = 0;
    virtual void flush() = 0;
    virtual void submitAndWait() = 0;
};

// Returns nullptr and sets error when no gfx950 device can be opened (factory convention of
// createVulkan / createGles).
std::unique_ptr<ComputeBackend> createHip(std::string& error);

inline int32_t floatBits(float f) {
    int32_t i;
    static_assert(sizeof i == sizeof f, "");
    __builtin_memcpy(&i, &f, 4);
    return i;
}

inline float bitsFloat(int32_t i) {
    float f;
    __builtin_memcpy(&f, &i, 4);
    return f;
}

}  // namespace neko::gpu
