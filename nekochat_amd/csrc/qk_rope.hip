// Qwen3 attention prologue for gfx950: per-head q/k RMSNorm fused with NeoX half-split RoPE, in
// place on the q and k heads of each qkv row (rope.comp:1-55; CPU qwen3_model.cpp:249-253 =
// cpu::rmsNorm per head, cpu_ops.cpp:502-511, then cpu::rope, cpu_ops.cpp:513-524).
//
// Fast path: one wavefront per token row. A head of hd elements is spread over L lanes; lane l
// holds the V elements [lV, lV+V) of the first half AND their NeoX partners [hd/2 + lV, ...), so the
// rotation needs no cross-lane exchange. 64/L heads are processed per wave pass and up to U passes
// are loaded before any is computed. The head's sum of squares (double, like the reference) is
// reduced over its L lanes with DPP only. The token's cos/sin row and the two norm weight vectors
// are loaded once per row and reused by every head. V heads are never touched.
//
// Fallback: one 64-thread workgroup per (head, row) staging the head in LDS (any even hd <= 512).
#include <cmath>

#include "internal.h"

namespace neko_hip {
namespace {

struct QkArgs {
    void* qkv;
    int64_t stride;
    int64_t rows;
    int n_q;
    int n_kv;
    int hd;
    int64_t pos0;
    const int32_t* positions;
    const float* wqk;  // q_norm[hd] | k_norm[hd], or null
    const float* cs;   // [n_pos][hd/2] (cos, sin)
    int64_t n_pos;
    float eps;
};

__device__ __forceinline__ bool row_position(const QkArgs& a, int64_t t, int64_t& pos) {
    pos = a.positions ? static_cast<int64_t>(a.positions[t]) : a.pos0 + t;
    return pos >= 0 && pos < a.n_pos;
}

template <typename T, int L, int V, int U>
__global__ __launch_bounds__(256) void qk_rope_kernel(QkArgs a) {
    constexpr int HPW = kWave / L;  // heads per wave pass
    typedef typename VecOf<T, V>::V VT;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (t >= a.rows) return;
    int64_t pos;
    if (!row_position(a, t, pos)) return;  // wave-uniform

    const int hl = lane % L;  // lane within its head
    const int hs = lane / L;  // head slot within the pass
    const int half = a.hd / 2;
    const int i0 = hl * V;  // first rotation pair of this lane

    float cv[V], sv[V];
    const float* csr = a.cs + pos * a.hd + 2 * i0;
#pragma unroll
    for (int e = 0; e < V; e++) {
        const float2v c = *reinterpret_cast<const float2v*>(csr + 2 * e);
        cv[e] = c[0];
        sv[e] = c[1];
    }
    const bool norm = a.wqk != nullptr;
    float wqa[V], wqb[V], wka[V], wkb[V];
#pragma unroll
    for (int e = 0; e < V; e++) {
        wqa[e] = norm ? a.wqk[i0 + e] : 1.0f;
        wqb[e] = norm ? a.wqk[half + i0 + e] : 1.0f;
        wka[e] = norm ? a.wqk[a.hd + i0 + e] : 1.0f;
        wkb[e] = norm ? a.wqk[a.hd + half + i0 + e] : 1.0f;
    }

    T* row = static_cast<T*>(a.qkv) + t * a.stride;
    const int nh = a.n_q + a.n_kv;
    for (int p0 = 0; p0 < nh; p0 += HPW * U) {
        VT va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int head = p0 + u * HPW + hs;
            va[u] = VT{};
            vb[u] = VT{};
            if (head < nh) {
                const T* hp = row + static_cast<int64_t>(head) * a.hd + i0;
                va[u] = *reinterpret_cast<const VT*>(hp);
                vb[u] = *reinterpret_cast<const VT*>(hp + half);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int head = p0 + u * HPW + hs;
            float fa[V], fb[V];
#pragma unroll
            for (int e = 0; e < V; e++) {
                if constexpr (V == 1) {
                    fa[e] = to_f32(va[u]);
                    fb[e] = to_f32(vb[u]);
                } else {
                    fa[e] = to_f32(va[u][e]);
                    fb[e] = to_f32(vb[u][e]);
                }
            }
            if (norm) {
                // Squares of f16/f32 values are exact in double, so fma == the reference's mul + add.
                double ss = 0.0;
#pragma unroll
                for (int e = 0; e < V; e++) {
                    ss = __builtin_fma(static_cast<double>(fa[e]), static_cast<double>(fa[e]), ss);
                    ss = __builtin_fma(static_cast<double>(fb[e]), static_cast<double>(fb[e]), ss);
                }
                ss = group_sum_f64<L>(ss);
                const float r = static_cast<float>(1.0 / sqrt(ss / a.hd + static_cast<double>(a.eps)));
                const bool is_q = head < a.n_q;
#pragma unroll
                for (int e = 0; e < V; e++) {
                    fa[e] = fa[e] * r * (is_q ? wqa[e] : wka[e]);
                    fb[e] = fb[e] * r * (is_q ? wqb[e] : wkb[e]);
                }
            }
            VT oa, ob;
#pragma unroll
            for (int e = 0; e < V; e++) {
                const float x0 = fa[e] * cv[e] - fb[e] * sv[e];
                const float x1 = fa[e] * sv[e] + fb[e] * cv[e];
                if constexpr (V == 1) {
                    oa = from_f32<T>(x0);
                    ob = from_f32<T>(x1);
                } else {
                    oa[e] = from_f32<T>(x0);
                    ob[e] = from_f32<T>(x1);
                }
            }
            if (head < nh) {
                T* hp = row + static_cast<int64_t>(head) * a.hd + i0;
                *reinterpret_cast<VT*>(hp) = oa;
                *reinterpret_cast<VT*>(hp + half) = ob;
            }
        }
    }
}

// Any even hd <= 512: one 64-thread workgroup per (head, row).
template <typename T>
__global__ __launch_bounds__(64) void qk_rope_generic(QkArgs a) {
    __shared__ float v[512];
    const int head = blockIdx.x;
    const int64_t t = blockIdx.y;
    int64_t pos;
    if (!row_position(a, t, pos)) return;
    T* hp = static_cast<T*>(a.qkv) + t * a.stride + static_cast<int64_t>(head) * a.hd;
    const int l = threadIdx.x;
    double ss = 0.0;
    for (int d = l; d < a.hd; d += 64) {
        const float x = to_f32(hp[d]);
        v[d] = x;
        ss += static_cast<double>(x) * static_cast<double>(x);
    }
    ss = wave_sum_f64(ss);
    __syncthreads();
    const bool norm = a.wqk != nullptr;
    const float r = norm ? static_cast<float>(1.0 / sqrt(ss / a.hd + static_cast<double>(a.eps))) : 1.0f;
    const float* wn = a.wqk + (head >= a.n_q ? a.hd : 0);
    const int half = a.hd / 2;
    const float* csr = a.cs + pos * a.hd;
    for (int i = l; i < half; i += 64) {
        float x0 = v[i], x1 = v[i + half];
        if (norm) {
            x0 = x0 * r * wn[i];
            x1 = x1 * r * wn[i + half];
        }
        const float c = csr[2 * i], s = csr[2 * i + 1];
        hp[i] = from_f32<T>(x0 * c - x1 * s);
        hp[i + half] = from_f32<T>(x0 * s + x1 * c);
    }
}

typedef void (*QkKernel)(QkArgs);

template <typename T, int V>
QkKernel pick_l(int L) {
    switch (L) {
        case 2: return qk_rope_kernel<T, 2, V, 8>;
        case 4: return qk_rope_kernel<T, 4, V, 8>;
        case 8: return qk_rope_kernel<T, 8, V, 8>;
        case 16: return qk_rope_kernel<T, 16, V, 4>;
        case 32: return qk_rope_kernel<T, 32, V, 4>;
        case 64: return qk_rope_kernel<T, 64, V, 4>;
    }
    return nullptr;
}

template <typename T>
QkKernel pick_lv(int L, int V) {
    switch (V) {
        case 1: return pick_l<T, 1>(L);
        case 2: return pick_l<T, 2>(L);
        case 4: return pick_l<T, 4>(L);
        case 8: return pick_l<T, 8>(L);
    }
    return nullptr;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_qk_norm_rope(neko_hip_ctx* ctx, void* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv,
                                     int hd, int64_t pos0, const int32_t* positions, const float* wqk, const float* cs,
                                     int64_t n_pos, float eps, int dtype) {
    const char* what = "neko_hip_qk_norm_rope";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && n_q >= 0 && n_kv >= 0 && hd > 0 && hd % 2 == 0 && hd <= 512 && n_pos >= 0,
                 "%s: bad shape rows=%lld n_q=%d n_kv=%d hd=%d n_pos=%lld", what, (long long)rows, n_q, n_kv, hd,
                 (long long)n_pos);
    const int nh = n_q + n_kv;
    if (rows == 0 || nh == 0 || n_pos == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, qkv && cs, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, row_stride >= static_cast<int64_t>(nh) * hd, "%s: row stride %lld < %d heads x %d", what,
                 (long long)row_stride, nh, hd);
    NEKO_REQUIRE(ctx, n_pos <= INT64_MAX / hd, "%s: n_pos too large", what);
    NEKO_REQUIRE(ctx, rows <= 0x7fffffffLL * 4, "%s: too many rows", what);

    const size_t esz = dtype_size(dtype);
    const int half = hd / 2;
    QkKernel k = nullptr;
    // Widest per-lane vector whose lane count per head is a power of two and whose loads stay aligned.
    for (int V = static_cast<int>(16 / esz); V >= 1 && !k; V /= 2) {
        if (half % V) continue;
        const int L = half / V;
        if (L < 2 || L > 64 || (L & (L - 1))) continue;
        const size_t vb = V * esz;
        if (!aligned(qkv, vb) || (row_stride * esz) % vb || (half * esz) % vb) continue;
        if (!aligned(cs, 8)) break;
        k = dtype == NEKO_DT_F16 ? pick_lv<half_t>(L, V) : pick_lv<float>(L, V);
    }
    if (k) {
        hipLaunchKernelGGL(k, dim3(static_cast<uint32_t>((rows + 3) / 4)), dim3(256), 0, ctx->stream,
                           QkArgs{qkv, row_stride, rows, n_q, n_kv, hd, pos0, positions, wqk, cs, n_pos, eps});
        return after_launch(ctx, what);
    }
    NEKO_REQUIRE(ctx, rows <= 65535 * 64LL, "%s: %lld rows exceed the fallback grid", what, (long long)rows);
    QkKernel g = dtype == NEKO_DT_F16 ? qk_rope_generic<half_t> : qk_rope_generic<float>;
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        const int64_t n = rows - r0 < 65535 ? rows - r0 : 65535;
        char* base = static_cast<char*>(qkv) + r0 * row_stride * static_cast<int64_t>(esz);
        const int32_t* pp = positions ? positions + r0 : nullptr;
        hipLaunchKernelGGL(g, dim3(static_cast<uint32_t>(nh), static_cast<uint32_t>(n)), dim3(64), 0, ctx->stream,
                           QkArgs{base, row_stride, n, n_q, n_kv, hd, pos0 + r0, pp, wqk, cs, n_pos, eps});
        if (int rc = after_launch(ctx, what)) return rc;
    }
    return NEKO_OK;
}
