// C ABI: contexts, streams, memory and error reporting (the ComputeBackend buffer / submission
// contract, gpu/compute.h:28-44, expressed as plain C over one in-order HIP stream per context).
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <unordered_map>

#include "internal.h"

namespace {
thread_local std::string g_create_error = "no error";
}

namespace neko_hip {

int fail(neko_hip_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    else g_create_error = buf;
    return code;
}

int check(neko_hip_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return NEKO_OK;
    return fail(ctx, NEKO_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int enter(neko_hip_ctx* ctx) {
    if (!ctx) return fail(nullptr, NEKO_ERR_INVALID, "null context");
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess || cur != ctx->device) return check(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    return NEKO_OK;
}

int after_launch(neko_hip_ctx* ctx, const char* what) { return check(ctx, hipGetLastError(), what); }

FastDiv make_fast_div(uint32_t d) {
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) s++;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
    return FastDiv{d, static_cast<uint32_t>(m), s};
}

int resident_blocks_per_cu(const void* kernel, int block, size_t lds_bytes) {
    // Keyed by kernel, block size and LDS (every device here is the same gfx950 part).
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t>, int> cache;
    std::lock_guard<std::mutex> lk(mu);
    const auto key = std::make_tuple(kernel, block, lds_bytes);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds_bytes) != hipSuccess || n < 1) {
        (void)hipGetLastError();
        n = 1;
    }
    cache.emplace(key, n);
    return n;
}

int64_t persistent_grid(neko_hip_ctx* ctx, const void* kernel, int block, int64_t work_blocks, size_t lds_bytes) {
    const int64_t cap =
        static_cast<int64_t>(ctx->cu_count > 0 ? ctx->cu_count : 256) * resident_blocks_per_cu(kernel, block, lds_bytes);
    return work_blocks < cap ? work_blocks : cap;
}

int capturing(neko_hip_ctx* ctx, hipStream_t stream, bool* yes) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &st);
    if (e == hipErrorStreamCaptureImplicit) {
        // The null stream, queried while another stream captures in global mode: it may not be used
        // either, which is what the callers need to know.
        (void)hipGetLastError();
        *yes = true;
        return NEKO_OK;
    }
    if (int rc = check(ctx, e, "hipStreamIsCapturing")) return rc;
    *yes = st != hipStreamCaptureStatusNone;
    return NEKO_OK;
}

int workspace(neko_hip_ctx* ctx, size_t bytes, void** out, int slot) {
    if (bytes > ctx->workspace_bytes[slot]) {
        // Growing allocates, which a stream under graph capture cannot record.
        bool cap = false;
        if (int rc = capturing(ctx, ctx->stream, &cap)) return rc;
        if (cap)
            return fail(ctx, NEKO_ERR_INVALID,
                        "matmul workspace must grow to %zu bytes (holds %zu) while the stream is being captured: make "
                        "one uncaptured call at the largest shape first, or capture neko_hip_matmul_noalloc",
                        bytes, ctx->workspace_bytes[slot]);
        // The next power of two (at least 1 MiB): the buffers a slot outgrows add up to less than the
        // one it has, however the requests rise.
        size_t grown = size_t(1) << 20;
        while (grown < bytes) grown <<= 1;
        void* p = nullptr;
        if (int rc = check(ctx, hipMalloc(&p, grown), "hipMalloc (workspace)")) return rc;
        // The old buffer is retired, not freed: queued work and graphs captured earlier still use it.
        if (ctx->workspace[slot]) ctx->retired.push_back(ctx->workspace[slot]);
        ctx->workspace[slot] = p;
        ctx->workspace_bytes[slot] = grown;
    }
    *out = ctx->workspace[slot];
    return NEKO_OK;
}

}  // namespace neko_hip

using namespace neko_hip;

extern "C" {

int neko_hip_create(int device, neko_hip_ctx** out) {
    if (!out) return fail(nullptr, NEKO_ERR_INVALID, "neko_hip_create: null output pointer");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return fail(nullptr, NEKO_ERR_NO_DEVICE, "neko_hip_create: no HIP device is visible");
    }
    if (device < 0 || device >= n)
        return fail(nullptr, NEKO_ERR_INVALID, "neko_hip_create: device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(nullptr, NEKO_ERR_HIP, "neko_hip_create: hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, NEKO_ERR_NO_DEVICE, "neko_hip_create: device %d is %s; this library is built for gfx950", device,
                    prop.gcnArchName);
    if (hipSetDevice(device) != hipSuccess) return fail(nullptr, NEKO_ERR_HIP, "neko_hip_create: hipSetDevice failed");
    auto* ctx = new neko_hip_ctx;
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount;
    ctx->max_alloc = prop.totalGlobalMem;
    ctx->name = prop.name;
    ctx->stream = nullptr;  // the device's null stream until the caller routes work elsewhere
    if (matmul_scratch_setup(ctx) != NEKO_OK) {
        const std::string msg = "neko_hip_create: " + ctx->err;
        delete ctx;
        return fail(nullptr, NEKO_ERR_HIP, "%s", msg.c_str());
    }
    *out = ctx;
    return NEKO_OK;
}

int neko_hip_destroy(neko_hip_ctx* ctx) {
    if (!ctx) return NEKO_OK;
    int rc = enter(ctx);
    if (rc == NEKO_OK) rc = check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    matmul_scratch_release(ctx);
    lt_release(ctx);
    for (void* p : ctx->allocs) (void)hipFree(p);
    for (void* p : ctx->workspace)
        if (p) (void)hipFree(p);
    for (void* p : ctx->retired) (void)hipFree(p);
    if (ctx->switch_event) (void)hipEventDestroy(ctx->switch_event);
    delete ctx;
    return rc;
}

const char* neko_hip_last_error(const neko_hip_ctx* ctx) { return ctx ? ctx->err.c_str() : g_create_error.c_str(); }

int neko_hip_device_name(neko_hip_ctx* ctx, char* buf, size_t buf_bytes) {
    NEKO_REQUIRE(ctx, ctx && buf && buf_bytes > 0, "neko_hip_device_name: null argument");
    std::snprintf(buf, buf_bytes, "%s", ctx->name.c_str());
    return NEKO_OK;
}

size_t neko_hip_max_buffer_bytes(const neko_hip_ctx* ctx) { return ctx ? ctx->max_alloc : 0; }

int neko_hip_set_matmul_library(neko_hip_ctx* ctx, int enable) {
    NEKO_REQUIRE(ctx, ctx, "neko_hip_set_matmul_library: null context");
    ctx->use_library = enable != 0;
    return NEKO_OK;
}

int neko_hip_set_stream(neko_hip_ctx* ctx, void* hip_stream) {
    NEKO_ENTER(ctx);
    const hipStream_t next = static_cast<hipStream_t>(hip_stream);
    if (next == ctx->stream) return NEKO_OK;
    // The new stream waits for the work already issued on the old one (on the device, not the
    // host): the context's calls share its split-K workspace, which that work may still be using.
    // Not when either stream is under graph capture: a capture cannot wait on work outside it, and
    // when its graph runs is up to the caller, who orders its launches.
    bool cap = false;
    if (int rc = capturing(ctx, next, &cap)) return rc;
    if (!cap)
        if (int rc = capturing(ctx, ctx->stream, &cap)) return rc;
    if (cap) {
        ctx->stream = next;
        return NEKO_OK;
    }
    if (!ctx->switch_event)
        if (int rc = check(ctx, hipEventCreateWithFlags(&ctx->switch_event, hipEventDisableTiming), "hipEventCreateWithFlags"))
            return rc;
    if (int rc = check(ctx, hipEventRecord(ctx->switch_event, ctx->stream), "hipEventRecord")) return rc;
    if (int rc = check(ctx, hipStreamWaitEvent(next, ctx->switch_event, 0), "hipStreamWaitEvent")) return rc;
    ctx->stream = next;
    return NEKO_OK;
}

void* neko_hip_get_stream(const neko_hip_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int neko_hip_alloc(neko_hip_ctx* ctx, size_t bytes, void** dev_ptr) {
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, dev_ptr != nullptr, "neko_hip_alloc: null output pointer");
    *dev_ptr = nullptr;
    void* p = nullptr;
    const int rc = check(ctx, hipMalloc(&p, bytes ? bytes : 16), "hipMalloc");
    if (rc != NEKO_OK) return rc;
    ctx->allocs.insert(p);
    *dev_ptr = p;
    return NEKO_OK;
}

int neko_hip_free(neko_hip_ctx* ctx, void* dev_ptr) {
    NEKO_ENTER(ctx);
    if (!dev_ptr) return NEKO_OK;
    NEKO_REQUIRE(ctx, ctx->allocs.count(dev_ptr) == 1, "neko_hip_free: %p was not allocated by this context", dev_ptr);
    // Work queued on the stream may still use the buffer.
    int rc = check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc != NEKO_OK) return rc;
    ctx->allocs.erase(dev_ptr);
    return check(ctx, hipFree(dev_ptr), "hipFree");
}

int neko_hip_upload(neko_hip_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes) {
    NEKO_ENTER(ctx);
    if (bytes == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, dst_dev && src_host, "neko_hip_upload: null pointer");
    int rc = check(ctx, hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
    if (rc != NEKO_OK) return rc;
    // The source is pageable host memory the caller may reuse as soon as this returns.
    return check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int neko_hip_download(neko_hip_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes) {
    NEKO_ENTER(ctx);
    if (bytes == 0) return check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    NEKO_REQUIRE(ctx, dst_host && src_dev, "neko_hip_download: null pointer");
    int rc = check(ctx, hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync D2H");
    if (rc != NEKO_OK) return rc;
    return check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int neko_hip_memset(neko_hip_ctx* ctx, void* dst_dev, int value, size_t bytes) {
    NEKO_ENTER(ctx);
    if (bytes == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, dst_dev != nullptr, "neko_hip_memset: null pointer");
    return check(ctx, hipMemsetAsync(dst_dev, value, bytes, ctx->stream), "hipMemsetAsync");
}

int neko_hip_synchronize(neko_hip_ctx* ctx) {
    NEKO_ENTER(ctx);
    return check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

}  // extern "C"
