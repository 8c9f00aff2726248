// Qwen3 attention prologue: argument checks, launch and the C entry points of the q/k RMSNorm +
// NeoX RoPE kernels (qk_rope_kernels.h), with and without the fused KV-cache store.
#include <algorithm>

#include "qk_rope_kernels.h"

namespace neko_hip {
namespace {

// 1 / hd when hd is a power of two (the scale then multiplies by it, exactly), else 0 (divide).
double inv_pow2(int hd) { return hd > 0 && (hd & (hd - 1)) == 0 ? 1.0 / hd : 0.0; }

// Shape and pointer checks shared by both entry points; *skip when there is nothing to do.
int qk_check(neko_hip_ctx* ctx, const char* what, const QkArgs& a, int dtype, bool* skip) {
    *skip = false;
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, a.rows >= 0 && a.n_q >= 0 && a.n_kv >= 0 && a.hd > 0 && a.hd % 2 == 0 && a.hd <= 512 && a.n_pos >= 0,
                 "%s: bad shape rows=%lld n_q=%d n_kv=%d hd=%d n_pos=%lld", what, (long long)a.rows, a.n_q, a.n_kv, a.hd,
                 (long long)a.n_pos);
    const int nh = a.n_q + a.n_kv;
    if (a.rows == 0 || nh == 0 || a.n_pos == 0) {
        *skip = true;
        return NEKO_OK;
    }
    NEKO_REQUIRE(ctx, a.qkv && a.cs, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, a.stride >= static_cast<int64_t>(nh) * a.hd, "%s: row stride %lld < %d heads x %d", what,
                 (long long)a.stride, nh, a.hd);
    NEKO_REQUIRE(ctx, a.n_pos <= INT64_MAX / a.hd, "%s: n_pos too large", what);
    NEKO_REQUIRE(ctx, a.rows <= 0x7fffffffLL * 4, "%s: too many rows", what);
    return NEKO_OK;
}

// Launches the op; with kv (a.k_cache set) the fused kernel when one fits, else *fused = false and
// only the q/k part ran.
int qk_launch(neko_hip_ctx* ctx, const char* what, QkArgs a, int dtype, bool kv, bool* fused) {
    *fused = false;
    const size_t esz = dtype_size(dtype);
    const int half = a.hd / 2;
    const int nqk = a.n_q + a.n_kv;
    QkKernel k = nullptr;
    bool with_kv = false;
    int split = 1;  // work items per token (the roll kernel's S)
    // Widest per-lane vector whose lane count per head is a power of two and whose loads stay aligned.
    const int vmax = static_cast<int>(16 / esz);
    for (int V = vmax; V >= 1 && !k; V /= 2) {
        if (half % V) continue;
        const int L = half / V;
        if (L < 2 || L > 64 || (L & (L - 1))) continue;
        const size_t vb = V * esz;
        if (!aligned(a.qkv, vb) || (a.stride * esz) % vb || (half * esz) % vb) continue;
        if (!aligned(a.cs, 8)) break;
        if (kv && aligned(a.k_cache, 2 * V) && aligned(a.v_cache, 2 * V)) {
            k = dtype == NEKO_DT_F16 ? pick_qk_f16(L, V, nqk + a.n_kv, true, &split)
                                     : pick_qk_f32(L, V, nqk + a.n_kv, true, &split);
            with_kv = k != nullptr;
        }
        if (!k) k = dtype == NEKO_DT_F16 ? pick_qk_f16(L, V, nqk, false, &split) : pick_qk_f32(L, V, nqk, false, &split);
    }
    if (!with_kv) a.k_cache = a.v_cache = nullptr;
    if (k) {
        // Persistent waves: as many workgroups as stay resident together, trimmed so that every wave
        // gets the same number of work items (ceil(items / resident waves)) and no partial last round
        // is left; a token is `split` items, and the wave count (4 x blocks) stays a multiple of it.
        // A wave takes at most kQkMaxTokensPerWave items (the roll kernel holds one position per
        // lane), so larger row counts go in several launches.
        NEKO_REQUIRE(ctx, split == 1 || split == 2, "%s: bad split %d", what, split);  // 4 x blocks is even
        const int64_t need = (a.rows * split + 3) / 4;
        int64_t blocks = persistent_grid(ctx, reinterpret_cast<const void*>(k), 256, need);
        const int64_t chunk = std::min<int64_t>(a.rows, 4 * blocks * kQkMaxTokensPerWave / split);
        if (blocks < need) {
            const int64_t items = chunk * split;
            const int64_t per = (items + 4 * blocks - 1) / (4 * blocks);
            blocks = ((items + per - 1) / per + 3) / 4;
        }
        for (int64_t r0 = 0; r0 < a.rows; r0 += chunk) {
            QkArgs s = a;
            s.rows = std::min(chunk, a.rows - r0);
            s.qkv = static_cast<char*>(a.qkv) + r0 * a.stride * static_cast<int64_t>(esz);
            if (a.positions) s.positions = a.positions + r0;
            else s.pos0 = a.pos0 + r0;
            const int64_t b = std::min<int64_t>(blocks, (s.rows * split + 3) / 4);
            hipLaunchKernelGGL(k, dim3(static_cast<uint32_t>(b)), dim3(256), 0, ctx->stream, s);
            if (int rc = after_launch(ctx, what)) return rc;
        }
        *fused = with_kv;
        return NEKO_OK;
    }
    NEKO_REQUIRE(ctx, a.rows <= 65535 * 64LL, "%s: %lld rows exceed the fallback grid", what, (long long)a.rows);
    QkKernel g = dtype == NEKO_DT_F16 ? qk_rope_generic<half_t> : qk_rope_generic<float>;
    const int64_t rows = a.rows;
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        QkArgs s = a;
        s.rows = rows - r0 < 65535 ? rows - r0 : 65535;
        s.qkv = static_cast<char*>(a.qkv) + r0 * a.stride * static_cast<int64_t>(esz);
        if (a.positions) s.positions = a.positions + r0;
        else s.pos0 = a.pos0 + r0;
        hipLaunchKernelGGL(g, dim3(static_cast<uint32_t>(nqk), static_cast<uint32_t>(s.rows)), dim3(64), 0, ctx->stream, s);
        if (int rc = after_launch(ctx, what)) return rc;
    }
    return NEKO_OK;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_qk_norm_rope(neko_hip_ctx* ctx, void* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv,
                                     int hd, int64_t pos0, const int32_t* positions, const float* wqk, const float* cs,
                                     int64_t n_pos, float eps, int dtype) {
    const char* what = "neko_hip_qk_norm_rope";
    NEKO_ENTER(ctx);
    const QkArgs a{qkv, row_stride, rows, n_q, n_kv, hd, pos0, positions, wqk, cs, n_pos, eps, nullptr, nullptr, inv_pow2(hd)};
    bool skip, fused;
    if (int rc = qk_check(ctx, what, a, dtype, &skip)) return rc;
    if (skip) return NEKO_OK;
    return qk_launch(ctx, what, a, dtype, false, &fused);
}

extern "C" int neko_hip_qk_norm_rope_kv(neko_hip_ctx* ctx, void* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv,
                                        int hd, int64_t pos0, const int32_t* positions, const float* wqk, const float* cs,
                                        int64_t n_pos, float eps, uint16_t* k_cache, uint16_t* v_cache, int64_t cache_rows,
                                        int dtype) {
    const char* what = "neko_hip_qk_norm_rope_kv";
    NEKO_ENTER(ctx);
    const QkArgs a{qkv, row_stride, rows, n_q, n_kv, hd, pos0, positions, wqk, cs, n_pos, eps, k_cache, v_cache, inv_pow2(hd)};
    bool skip, fused;
    if (int rc = qk_check(ctx, what, a, dtype, &skip)) return rc;
    if (skip) return NEKO_OK;
    NEKO_REQUIRE(ctx, n_kv > 0 && k_cache && v_cache, "%s: the KV store needs n_kv > 0 and both caches", what);
    NEKO_REQUIRE(ctx, cache_rows >= n_pos, "%s: cache_rows %lld < n_pos %lld (every valid position needs a cache row)",
                 what, (long long)cache_rows, (long long)n_pos);
    const int64_t kvw = static_cast<int64_t>(n_kv) * hd;
    NEKO_REQUIRE(ctx, row_stride >= static_cast<int64_t>(n_q) * hd + 2 * kvw, "%s: row stride %lld holds no v heads", what,
                 (long long)row_stride);
    NEKO_REQUIRE(ctx, cache_rows <= (int64_t(1) << 60) / kvw, "%s: cache too large", what);
    const size_t sq = rows_span(rows, static_cast<int64_t>(n_q) * hd + 2 * kvw, row_stride, dtype_size(dtype));
    const size_t sc = static_cast<size_t>(cache_rows * kvw) * 2;
    NEKO_REQUIRE(ctx, sq != 0, "%s: qkv rows span more than 2^62 bytes", what);
    NEKO_REQUIRE(ctx, !overlaps(k_cache, sc, v_cache, sc) && !overlaps(qkv, sq, k_cache, sc) && !overlaps(qkv, sq, v_cache, sc),
                 "%s: the caches may not overlap each other or qkv", what);
    if (int rc = qk_launch(ctx, what, a, dtype, true, &fused)) return rc;
    if (fused) return NEKO_OK;
    // No fused kernel for this shape: the same result from the two ops in order. Rows outside the
    // RoPE table were left untouched; the store skips them because cache row = position and
    // positions beyond n_pos are excluded by clamping the cache to n_pos rows.
    return launch_store_kv(ctx, what, qkv, row_stride, static_cast<int64_t>(n_q) * hd, static_cast<int64_t>(n_q) * hd + kvw,
                           rows, kvw, pos0, positions, k_cache, v_cache, n_pos, dtype);
}
