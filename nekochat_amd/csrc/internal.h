// Host-side internals shared by the C-ABI translation units: the context, status helpers and the
// launch-time checks every entry point runs.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>
#include <unordered_set>
#include <vector>

#include "../../include/neko_hip.h"
#include "device.h"

namespace neko_hip {
struct LtState;  // hipBLASLt handle and per-shape plans (matmul_lib.hip)
}

struct neko_hip_ctx {
    int device = -1;
    hipStream_t stream = nullptr;  // null = the device's null stream
    int cu_count = 0;
    size_t max_alloc = 0;
    std::string name;
    std::string err;
    std::unordered_set<void*> allocs;
    // Device scratch, grown on demand: [0] split-K partial sums, [1] the f32-activation matmul's f16
    // planes and sums (its GEMMs may split K into [0] meanwhile).
    void* workspace[2] = {nullptr, nullptr};
    size_t workspace_bytes[2] = {0, 0};
    std::vector<void*> retired;  // outgrown workspaces, kept until destroy (captured graphs may use them)
    hipEvent_t switch_event = nullptr;  // orders a newly routed stream after the previous one
    void* scratch = nullptr;  // device address of the matmul's fixed split-K scratch on this device
    neko_hip::LtState* lt = nullptr;  // created by the first matmul that takes hipBLASLt
    bool use_library = true;          // neko_hip_set_matmul_library
};

namespace neko_hip {

// Records a formatted message on ctx (or the thread-wide create error when ctx is null) and
// returns code.
int fail(neko_hip_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
// NEKO_OK, or NEKO_ERR_HIP with the HIP error string and the failing call named.
int check(neko_hip_ctx* ctx, hipError_t e, const char* what);
// Validates ctx and makes its device current for this thread.
int enter(neko_hip_ctx* ctx);
// Picks up launch errors of the kernel just enqueued.
int after_launch(neko_hip_ctx* ctx, const char* what);

FastDiv make_fast_div(uint32_t d);

// The context's device workspace `slot` (0 or 1), at least `bytes` long, shared by every op on ctx.
// Grown on demand to the next power of two; an outgrown buffer stays allocated until
// neko_hip_destroy, since queued work and captured graphs may still use it -- the doubling keeps all
// retired buffers of a slot together smaller than its live one. Growing while ctx's stream is under
// graph capture fails (NEKO_ERR_INVALID).
int workspace(neko_hip_ctx* ctx, size_t bytes, void** out, int slot = 0);
// Looks up (once per device, with that device current) and records in ctx the device address of
// the fixed scratch array that neko_hip_matmul_noalloc uses (matmul.hip).
int matmul_scratch_setup(neko_hip_ctx* ctx);
// The plain F16 weight matmul (f16 activations) on hipBLASLt: *done = true when the library ran it;
// false (NEKO_OK) when it has no algorithm for the shape, or the library could not be initialised --
// the caller then runs its own kernels.
int lt_matmul(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w, int64_t row_bytes,
              int64_t N, const float* bias, void* y, int64_t y_stride, int flags, int y_dtype, bool* done);
// Frees ctx's hipBLASLt handle and plans (neko_hip_destroy, after its stream has drained).
void lt_release(neko_hip_ctx* ctx);
// Gives up ctx's claim on its device's scratch array (taken by its first neko_hip_matmul_noalloc
// call), once its stream has drained.
void matmul_scratch_release(const neko_hip_ctx* ctx);
// Whether `stream` is under graph capture.
int capturing(neko_hip_ctx* ctx, hipStream_t stream, bool* yes);

// Workgroups of `block` threads of `kernel` that fit on one CU at once (cached per kernel), and the
// grid of a persistent kernel: that many per CU, or fewer when there is less work.
int resident_blocks_per_cu(const void* kernel, int block, size_t lds_bytes = 0);
int64_t persistent_grid(neko_hip_ctx* ctx, const void* kernel, int block, int64_t work_blocks, size_t lds_bytes = 0);

// The KV-cache store's launch (kv_store.hip), after argument checks; also the second half of the
// unfused q/k RoPE + KV store path.
int launch_store_kv(neko_hip_ctx* ctx, const char* what, const void* qkv, int64_t row_stride, int64_t k_off, int64_t v_off,
                    int64_t rows, int64_t width, int64_t pos0, const int32_t* positions, uint16_t* k_cache,
                    uint16_t* v_cache, int64_t cache_rows, int dtype);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Byte ranges [a, a + an) and [b, b + bn) share a byte.
inline bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return an && bn && pa < pb + bn && pb < pa + an;
}
// Bytes from the first element of `rows` rows of `width` elements, `stride` elements apart, to the
// end of the last; 0 when that does not fit in 62 bits (callers reject it).
inline size_t rows_span(int64_t rows, int64_t width, int64_t stride, size_t esz) {
    if (rows <= 0 || width <= 0) return 0;
    if (stride > 0 && rows - 1 > ((int64_t(1) << 62) - width) / stride) return 0;
    return static_cast<size_t>((rows - 1) * stride + width) * esz;
}
// An op that reads rows at `in` and writes rows at `out` (same shape) is well defined when the two
// are the same rows -- same address and stride, each row rewritten in place by the code that read
// it -- or share no byte. Any other overlap would let one row's store land on a row another wave
// is still reading.
inline bool same_or_disjoint(const void* in, int64_t in_stride, const void* out, int64_t out_stride, size_t span_in,
                             size_t span_out) {
    return (in == out && in_stride == out_stride) || !overlaps(in, span_in, out, span_out);
}
inline size_t dtype_size(int dtype) { return dtype == NEKO_DT_F16 ? 2 : 4; }
inline bool valid_dtype(int dtype) { return dtype == NEKO_DT_F16 || dtype == NEKO_DT_F32; }

}  // namespace neko_hip

#define NEKO_ENTER(ctx)                          \
    do {                                         \
        const int neko_rc_ = neko_hip::enter(ctx); \
        if (neko_rc_ != NEKO_OK) return neko_rc_; \
    } while (0)

#define NEKO_REQUIRE(ctx, cond, ...)                                        \
    do {                                                                    \
        if (!(cond)) return neko_hip::fail(ctx, NEKO_ERR_INVALID, __VA_ARGS__); \
    } while (0)
