// Elementwise activations for gfx950: SwiGLU (cpu_ops.cpp:526-533, silu_mul.comp) and GELU, tanh
// form (cpu_ops.cpp:20-23).
//
// Both are pure HBM streams. The (row, 16-byte chunk) space is flattened so that consecutive lanes
// take consecutive chunks of a row (fully coalesced loads and stores, no idle lanes at row ends).
// One chunk per thread and many small workgroups keep the most loads in flight (measured on MI355X:
// 1 item/thread beats 2 and 4 by 3-10%); loads are non-temporal (streamed once), stores are plain.
// Row/column come from a multiply-high division by the invariant chunks-per-row.
#include <cmath>

#include "internal.h"

namespace neko_hip {
namespace {

// SwiGLU element: silu(gate) * up in float, the SiLU from silu_fast (device.h): the libm form (expf
// and an IEEE division) made the stream VALU-bound (94% VALUBusy).
__device__ __forceinline__ float swiglu_ref(float gate, float up) { return silu_fast(gate) * up; }

// SwiGLU loads are non-temporal (measured faster), stores plain.
template <typename V>
__device__ __forceinline__ V swiglu_load(const V* p) {
    return load_nt(p);
}
template <typename V>
__device__ __forceinline__ void swiglu_store(V* p, V v) {
    *p = v;
}

// GELU: gelu_ref (device.h).

template <typename VT, typename T, int N>
__device__ __forceinline__ T lane_elem(const VT& v, int e) {
    if constexpr (N == 1) return v;
    else return v[e];
}

template <typename VT, typename T, int N>
__device__ __forceinline__ void set_elem(VT& v, int e, T x) {
    if constexpr (N == 1) v = x;
    else v[e] = x;
}

struct SwigluArgs {
    const void* h;
    int64_t hs;
    void* out;
    int64_t os;
    int64_t I;
    uint32_t items;  // rows * chunks per row, < 2^31
    FastDiv cpr;     // chunks per row
};

template <typename T, int N, int ITEMS>
__global__ __launch_bounds__(256) void swiglu_kernel(SwigluArgs a) {
    typedef typename VecOf<T, N>::V VT;
    // Runs of 128 workgroups' data per XCD (xcd_block): 1.8% faster at [8192, 9728] than launch order.
    const uint32_t base = xcd_block<128>(blockIdx.x, gridDim.x) * (256u * ITEMS) + threadIdx.x;
    VT g[ITEMS], u[ITEMS];
    int64_t src[ITEMS], dst[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const uint32_t idx = base + k * 256u;
        g[k] = VT{};
        u[k] = VT{};
        src[k] = dst[k] = -1;
        if (idx < a.items) {
            const uint32_t row = fast_div(idx, a.cpr);
            const int64_t col = static_cast<int64_t>(idx - row * a.cpr.d) * N;
            src[k] = row * a.hs + col;
            dst[k] = row * a.os + col;
            const T* hp = static_cast<const T*>(a.h) + src[k];
            g[k] = swiglu_load(reinterpret_cast<const VT*>(hp));
            u[k] = swiglu_load(reinterpret_cast<const VT*>(hp + a.I));
        }
    }
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        if (dst[k] < 0) continue;
        VT o;
#pragma unroll
        for (int e = 0; e < N; e++) {
            const float v = swiglu_ref(to_f32(lane_elem<VT, T, N>(g[k], e)), to_f32(lane_elem<VT, T, N>(u[k], e)));
            set_elem<VT, T, N>(o, e, from_f32<T>(v));
        }
        swiglu_store(reinterpret_cast<VT*>(static_cast<T*>(a.out) + dst[k]), o);
    }
}

template <typename T, int N, int ITEMS>
__global__ __launch_bounds__(256) void gelu_kernel(const T* x, T* y, int64_t n_chunks) {
    typedef typename VecOf<T, N>::V VT;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * ITEMS) + threadIdx.x;
    VT v[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t c = base + k * 256;
        v[k] = VT{};
        if (c < n_chunks) v[k] = load_nt(reinterpret_cast<const VT*>(x) + c);
    }
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t c = base + k * 256;
        if (c >= n_chunks) continue;
        VT o;
#pragma unroll
        for (int e = 0; e < N; e++) set_elem<VT, T, N>(o, e, from_f32<T>(gelu_ref(to_f32(lane_elem<VT, T, N>(v[k], e)))));
        reinterpret_cast<VT*>(y)[c] = o;
    }
}

constexpr int kItems = 1;

template <typename T, int N>
int launch_swiglu(neko_hip_ctx* ctx, const T* h, int64_t hs, T* out, int64_t os, int64_t rows, int64_t I) {
    const int64_t cpr = I / N;
    // Row slices keep every flattened chunk index below 2^31.
    const int64_t slice = (int64_t(1) << 31) / cpr;
    for (int64_t r0 = 0; r0 < rows; r0 += slice) {
        const int64_t n = rows - r0 < slice ? rows - r0 : slice;
        const uint32_t items = static_cast<uint32_t>(n * cpr);
        SwigluArgs a{h + r0 * hs, hs, out + r0 * os, os, I, items, make_fast_div(static_cast<uint32_t>(cpr))};
        const uint32_t blocks = (items + 256u * kItems - 1) / (256u * kItems);
        hipLaunchKernelGGL((swiglu_kernel<T, N, kItems>), dim3(blocks), dim3(256), 0, ctx->stream, a);
        if (int rc = after_launch(ctx, "neko_hip_swiglu")) return rc;
    }
    return NEKO_OK;
}

template <typename T, int N>
int launch_gelu(neko_hip_ctx* ctx, const T* x, T* y, int64_t n_chunks) {
    if (n_chunks == 0) return NEKO_OK;
    const int64_t blocks = (n_chunks + 256 * kItems - 1) / (256 * kItems);
    if (blocks > 0x7fffffff) return fail(ctx, NEKO_ERR_UNSUPPORTED, "neko_hip_gelu_tanh: too many elements");
    hipLaunchKernelGGL((gelu_kernel<T, N, kItems>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, ctx->stream, x, y,
                       n_chunks);
    return after_launch(ctx, "neko_hip_gelu_tanh");
}

template <typename T>
int swiglu_typed(neko_hip_ctx* ctx, const void* h, int64_t hs, void* out, int64_t os, int64_t rows, int64_t I) {
    constexpr int N = Chunk16<T>::N;
    const T* hp = static_cast<const T*>(h);
    T* op = static_cast<T*>(out);
    const bool vec = I % N == 0 && hs % N == 0 && os % N == 0 && aligned(h, 16) && aligned(out, 16);
    return vec ? launch_swiglu<T, N>(ctx, hp, hs, op, os, rows, I) : launch_swiglu<T, 1>(ctx, hp, hs, op, os, rows, I);
}

template <typename T>
int gelu_typed(neko_hip_ctx* ctx, const void* x, void* y, int64_t n) {
    constexpr int N = Chunk16<T>::N;
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    if (!aligned(x, 16) || !aligned(y, 16)) return launch_gelu<T, 1>(ctx, xp, yp, n);
    const int64_t nc = n / N;
    if (int rc = launch_gelu<T, N>(ctx, xp, yp, nc)) return rc;
    return launch_gelu<T, 1>(ctx, xp + nc * N, yp + nc * N, n - nc * N);
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" {

int neko_hip_swiglu(neko_hip_ctx* ctx, const void* h, int64_t h_stride, void* out, int64_t out_stride, int64_t rows,
                    int64_t I, int dtype) {
    const char* what = "neko_hip_swiglu";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && I > 0 && I < (int64_t(1) << 31), "%s: bad shape rows=%lld I=%lld", what, (long long)rows,
                 (long long)I);
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, h && out, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, h_stride >= 2 * I && out_stride >= I, "%s: strides (%lld, %lld) too small for I=%lld", what,
                 (long long)h_stride, (long long)out_stride, (long long)I);
    // out over the gate halves of h (same pointer and stride: each chunk is rewritten by the thread
    // that read it) or disjoint from h.
    const size_t esz = dtype_size(dtype);
    const size_t sh = rows_span(rows, 2 * I, h_stride, esz), so = rows_span(rows, I, out_stride, esz);
    NEKO_REQUIRE(ctx, sh && so, "%s: rows span more than 2^62 bytes", what);
    NEKO_REQUIRE(ctx, (out == h && out_stride == h_stride) || !overlaps(h, sh, out, so),
                 "%s: out overlaps h without being its gate halves (same pointer and stride)", what);
    return dtype == NEKO_DT_F16 ? swiglu_typed<half_t>(ctx, h, h_stride, out, out_stride, rows, I)
                                : swiglu_typed<float>(ctx, h, h_stride, out, out_stride, rows, I);
}

int neko_hip_gelu_tanh(neko_hip_ctx* ctx, const void* x, void* y, int64_t n, int dtype) {
    const char* what = "neko_hip_gelu_tanh";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, n >= 0, "%s: negative size", what);
    if (n == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, x && y, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, n <= (int64_t(1) << 60), "%s: too many elements", what);
    const size_t bytes = static_cast<size_t>(n) * dtype_size(dtype);
    NEKO_REQUIRE(ctx, x == y || !overlaps(x, bytes, y, bytes), "%s: x and y overlap without being the same array", what);
    return dtype == NEKO_DT_F16 ? gelu_typed<half_t>(ctx, x, y, n) : gelu_typed<float>(ctx, x, y, n);
}

}  // extern "C"
