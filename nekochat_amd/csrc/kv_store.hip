// KV-cache store for gfx950 (cpu::storeKv, cpu_ops.cpp:535-542; GPU kv_store.comp:1-21): the k and v
// values of each row, written as f16 into cache row = the row's position.
//
// A pure stream: the (row, 8-element chunk) space is flattened so consecutive lanes take consecutive
// chunks of a row; each thread moves one chunk of k and one of v (16-byte f16 stores; f16 input is
// copied bit for bit, f32 input is rounded once to f16 with RNE, as toHalf does). Rows whose cache
// row is outside [0, cache_rows) are skipped. Odd widths or unaligned operands take a per-element
// kernel.
#include "internal.h"

namespace neko_hip {
namespace {

struct KvArgs {
    const void* qkv;
    int64_t stride;
    int64_t k_off;
    int64_t v_off;
    int64_t pos0;
    const int32_t* positions;
    uint16_t* kc;
    uint16_t* vc;
    int64_t width;
    int64_t cache_rows;
    uint32_t items;  // rows * chunks per row (< 2^31)
    FastDiv cpr;     // chunks per row
};

__device__ __forceinline__ int64_t cache_row(const KvArgs& a, int64_t t) {
    return a.positions ? static_cast<int64_t>(a.positions[t]) : a.pos0 + t;
}

// 8 values of T from p as 8 halves.
template <typename T>
__device__ __forceinline__ half8 load8_as_f16(const T* p) {
    if constexpr (sizeof(T) == 2) {
        return load_nt(reinterpret_cast<const half8*>(p));
    } else {
        const float4v lo = load_nt(reinterpret_cast<const float4v*>(p));
        const float4v hi = load_nt(reinterpret_cast<const float4v*>(p + 4));
        half8 h;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = static_cast<half_t>(lo[e]);
            h[4 + e] = static_cast<half_t>(hi[e]);
        }
        return h;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void store_kv_kernel(KvArgs a) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= a.items) return;
    const uint32_t t = fast_div(idx, a.cpr);
    const int64_t c = static_cast<int64_t>(idx - t * a.cpr.d) * 8;
    const int64_t p = cache_row(a, t);
    if (p < 0 || p >= a.cache_rows) return;
    const T* row = static_cast<const T*>(a.qkv) + static_cast<int64_t>(t) * a.stride;
    const half8 k = load8_as_f16(row + a.k_off + c);
    const half8 v = load8_as_f16(row + a.v_off + c);
    *reinterpret_cast<half8*>(a.kc + p * a.width + c) = k;
    *reinterpret_cast<half8*>(a.vc + p * a.width + c) = v;
}

// Any width and alignment: one thread per (row, element).
template <typename T>
__global__ __launch_bounds__(256) void store_kv_generic(KvArgs a, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const int64_t t = i / a.width, c = i - t * a.width;
    const int64_t p = cache_row(a, t);
    if (p < 0 || p >= a.cache_rows) return;
    const T* row = static_cast<const T*>(a.qkv) + t * a.stride;
    reinterpret_cast<half_t*>(a.kc)[p * a.width + c] = static_cast<half_t>(row[a.k_off + c]);
    reinterpret_cast<half_t*>(a.vc)[p * a.width + c] = static_cast<half_t>(row[a.v_off + c]);
}

template <typename T>
int launch_typed(neko_hip_ctx* ctx, const char* what, KvArgs a, int64_t rows) {
    const size_t esz = sizeof(T);
    const bool vec = a.width % 8 == 0 && aligned(a.qkv, 16) && (a.stride * esz) % 16 == 0 && (a.k_off * esz) % 16 == 0 &&
                     (a.v_off * esz) % 16 == 0 && aligned(a.kc, 16) && aligned(a.vc, 16);
    if (vec) {
        const int64_t cpr = a.width / 8;
        const int64_t slice = (int64_t(1) << 31) / cpr;  // rows per launch, keeping chunk indices < 2^31
        for (int64_t r0 = 0; r0 < rows; r0 += slice) {
            const int64_t n = rows - r0 < slice ? rows - r0 : slice;
            KvArgs s = a;
            s.qkv = static_cast<const T*>(a.qkv) + r0 * a.stride;
            if (a.positions) s.positions = a.positions + r0;
            else s.pos0 = a.pos0 + r0;
            s.items = static_cast<uint32_t>(n * cpr);
            s.cpr = make_fast_div(static_cast<uint32_t>(cpr));
            hipLaunchKernelGGL(store_kv_kernel<T>, dim3((s.items + 255u) / 256u), dim3(256), 0, ctx->stream, s);
            if (int rc = after_launch(ctx, what)) return rc;
        }
        return NEKO_OK;
    }
    const int64_t n = rows * a.width;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: too many elements for the fallback", what);
    hipLaunchKernelGGL(store_kv_generic<T>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, ctx->stream, a, n);
    return after_launch(ctx, what);
}

}  // namespace

int launch_store_kv(neko_hip_ctx* ctx, const char* what, const void* qkv, int64_t row_stride, int64_t k_off, int64_t v_off,
                    int64_t rows, int64_t width, int64_t pos0, const int32_t* positions, uint16_t* k_cache,
                    uint16_t* v_cache, int64_t cache_rows, int dtype) {
    KvArgs a{qkv, row_stride, k_off, v_off, pos0, positions, k_cache, v_cache, width, cache_rows, 0, FastDiv{}};
    return dtype == NEKO_DT_F16 ? launch_typed<half_t>(ctx, what, a, rows) : launch_typed<float>(ctx, what, a, rows);
}

}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_store_kv(neko_hip_ctx* ctx, const void* qkv, int64_t row_stride, int64_t k_off, int64_t v_off,
                                 int64_t rows, int64_t width, int64_t pos0, const int32_t* positions, uint16_t* k_cache,
                                 uint16_t* v_cache, int64_t cache_rows, int dtype) {
    const char* what = "neko_hip_store_kv";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && width > 0 && k_off >= 0 && v_off >= 0 && cache_rows >= 0,
                 "%s: bad shape rows=%lld width=%lld k_off=%lld v_off=%lld cache_rows=%lld", what, (long long)rows,
                 (long long)width, (long long)k_off, (long long)v_off, (long long)cache_rows);
    if (rows == 0 || cache_rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, qkv && k_cache && v_cache, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, row_stride >= k_off + width && row_stride >= v_off + width,
                 "%s: k/v columns [%lld, +%lld) / [%lld, +%lld) exceed the row stride %lld", what, (long long)k_off,
                 (long long)width, (long long)v_off, (long long)width, (long long)row_stride);
    NEKO_REQUIRE(ctx, cache_rows <= (int64_t(1) << 60) / width, "%s: cache too large", what);
    const size_t sq = rows_span(rows, (k_off > v_off ? k_off : v_off) + width, row_stride, dtype_size(dtype));
    const size_t sc = static_cast<size_t>(cache_rows * width) * 2;
    NEKO_REQUIRE(ctx, sq != 0, "%s: qkv rows span more than 2^62 bytes", what);
    NEKO_REQUIRE(ctx, !overlaps(k_cache, sc, v_cache, sc) && !overlaps(qkv, sq, k_cache, sc) && !overlaps(qkv, sq, v_cache, sc),
                 "%s: the caches may not overlap each other or qkv", what);
    return launch_store_kv(ctx, what, qkv, row_stride, k_off, v_off, rows, width, pos0, positions, k_cache, v_cache,
                           cache_rows, dtype);
}
