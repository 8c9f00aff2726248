// Embedding gather with fused row dequantisation for gfx950 (embed.comp:1-51,
// QMatrix::dequantizeRow quant.cpp:230-253, GPT-2 wte + wpe gpt2_model.cpp:182-187).
//
// One wavefront per token. Each lane takes one 16-byte chunk of the stored row per step:
//   F16: 8 halves;  FP8: 16 codes sharing one block scale;  FP4: one whole 32-weight block
//   (weight j in the low nibble of byte j, weight 16 + j in the high nibble).
// Codes are decoded with the reference's bit trick (the code's bits placed into an f16 pattern that
// equals value / 256 for E4M3 or value / 16384 for E2M1, subnormals included), then multiplied in
// f32 by scale * 256 (or * 16384). Every such product has at most 15 significant bits, so it is
// exact and identical to the reference's f32 value; f16 output is one RNE rounding of it. This
// keeps the reference's 0x7F / 0xFF = +-480 (not NaN) and -0 codes. With wpe the position row is
// added in f32 first, then rounded once, as the reference does.
#include "internal.h"

namespace neko_hip {
namespace {

struct EmbedArgs {
    const int32_t* tokens;
    int64_t T;
    const uint8_t* table;
    int64_t row_bytes;
    int C;
    int64_t row_base;
    int64_t rows;
    const half_t* wpe;
    int64_t pos0;
    void* out;
    int64_t out_stride;
};

__device__ __forceinline__ float half_bits_to_f32(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(bits16)));
}

// Two E4M3 codes in bits [7:0] and [15:8] of w -> their f16 patterns (value / 256) as f32.
__device__ __forceinline__ void fp8_pair(uint32_t w, float& f0, float& f1) {
    const uint32_t c0 = w & 0xffu, c1 = (w >> 8) & 0xffu;
    f0 = half_bits_to_f32(((c0 & 0x80u) << 8) | ((c0 & 0x7fu) << 7));
    f1 = half_bits_to_f32(((c1 & 0x80u) << 8) | ((c1 & 0x7fu) << 7));
}

// E2M1 code in bits [3:0] of n -> its f16 pattern (value / 16384) as f32.
__device__ __forceinline__ float fp4_code(uint32_t n) { return half_bits_to_f32(((n & 8u) << 12) | ((n & 7u) << 9)); }

template <typename TO, int M>
__device__ __forceinline__ void store_out(TO* dst, const float (&v)[M]) {
    // M f32 results -> M outputs, written as 16-byte vectors.
    constexpr int PER = 16 / sizeof(TO);
#pragma unroll
    for (int q = 0; q < M / PER; q++) {
        typedef typename VecOf<TO, PER>::V VO;
        VO o;
#pragma unroll
        for (int e = 0; e < PER; e++) o[e] = from_f32<TO>(v[q * PER + e]);
        store_nt(reinterpret_cast<VO*>(dst) + q, o);
    }
}

template <int M>
__device__ __forceinline__ void add_wpe(float (&v)[M], const half_t* pe) {
    // M consecutive position values (M multiple of 8), 16-byte loads.
#pragma unroll
    for (int q = 0; q < M / 8; q++) {
        const half8 h = *reinterpret_cast<const half8*>(pe + 8 * q);
#pragma unroll
        for (int e = 0; e < 8; e++) v[8 * q + e] = v[8 * q + e] + static_cast<float>(h[e]);
    }
}

// Vector path. FMT: 0 F16, 1 FP8, 2 FP4. Requires C % 32 == 0 for FP8/FP4, C % 8 == 0 for F16, and
// 16-byte aligned rows everywhere.
template <int FMT, typename TO, bool WPE>
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (t >= a.T) return;
    const int64_t r = static_cast<int64_t>(a.tokens[t]) - a.row_base;
    if (r < 0 || r >= a.rows) return;  // another chunk of the table owns this token
    const uint8_t* row = a.table + r * a.row_bytes;
    TO* out = static_cast<TO*>(a.out) + t * a.out_stride;
    const half_t* pe = WPE ? a.wpe + (a.pos0 + t) * a.C : nullptr;

    if constexpr (FMT == 0) {
        const int nch = a.C / 8;
        constexpr int B = 4;  // chunks in flight per lane
        for (int j0 = 0; j0 < nch; j0 += B * kWave) {
            half8 h[B];
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j < nch) h[b] = *reinterpret_cast<const half8*>(row + 16 * j);
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j >= nch) continue;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = static_cast<float>(h[b][e]);
                if constexpr (WPE) add_wpe<8>(v, pe + 8 * j);
                store_out<TO, 8>(out + 8 * j, v);
            }
        }
    } else if constexpr (FMT == 1) {
        const int nch = a.C / 16;  // 16 codes per chunk, two chunks per block scale
        const uint8_t* scales = row + a.C;
        constexpr int B = 2;
        for (int j0 = 0; j0 < nch; j0 += B * kWave) {
            uint4v q[B];
            float s[B];
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j < nch) {
                    q[b] = *reinterpret_cast<const uint4v*>(row + 16 * j);
                    const half_t sh = *reinterpret_cast<const half_t*>(scales + 2 * (j >> 1));
                    s[b] = static_cast<float>(sh) * 256.0f;
                }
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j >= nch) continue;
                float v[16];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    float f0, f1, f2, f3;
                    fp8_pair(q[b][w], f0, f1);
                    fp8_pair(q[b][w] >> 16, f2, f3);
                    v[4 * w + 0] = f0 * s[b];
                    v[4 * w + 1] = f1 * s[b];
                    v[4 * w + 2] = f2 * s[b];
                    v[4 * w + 3] = f3 * s[b];
                }
                if constexpr (WPE) add_wpe<16>(v, pe + 16 * j);
                store_out<TO, 16>(out + 16 * j, v);
            }
        }
    } else {
        const int nb = a.C / 32;  // one 16-byte block per chunk
        const uint8_t* scales = row + a.C / 2;
        constexpr int B = 2;
        for (int j0 = 0; j0 < nb; j0 += B * kWave) {
            uint4v q[B];
            float s[B];
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j < nb) {
                    q[b] = *reinterpret_cast<const uint4v*>(row + 16 * j);
                    const half_t sh = *reinterpret_cast<const half_t*>(scales + 2 * j);
                    s[b] = static_cast<float>(sh) * 16384.0f;
                }
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int j = j0 + b * kWave + lane;
                if (j >= nb) continue;
                float lo[16], hi[16];
#pragma unroll
                for (int w = 0; w < 4; w++) {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t byte = (q[b][w] >> (8 * k)) & 0xffu;
                        lo[4 * w + k] = fp4_code(byte) * s[b];
                        hi[4 * w + k] = fp4_code(byte >> 4) * s[b];
                    }
                }
                if constexpr (WPE) {
                    add_wpe<16>(lo, pe + 32 * j);
                    add_wpe<16>(hi, pe + 32 * j + 16);
                }
                store_out<TO, 16>(out + 32 * j, lo);
                store_out<TO, 16>(out + 32 * j + 16, hi);
            }
        }
    }
}

// Any layout: one thread per element, byte addressing (the embed.comp scheme).
template <typename TO>
__global__ __launch_bounds__(256) void embed_generic(EmbedArgs a, int fmt, int use_wpe) {
    const int64_t t = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.C) return;
    const int64_t r = static_cast<int64_t>(a.tokens[t]) - a.row_base;
    if (r < 0 || r >= a.rows) return;
    const uint8_t* row = a.table + r * a.row_bytes;
    float v;
    if (fmt == 0) {
        v = half_bits_to_f32(row[2 * c] | (row[2 * c + 1] << 8));
    } else {
        const int b = c / 32;
        const uint8_t* sp = row + (fmt == 1 ? a.C : a.C / 2) + 2 * b;
        const float sc = half_bits_to_f32(sp[0] | (sp[1] << 8));
        if (fmt == 1) {
            const uint32_t code = row[c];
            v = half_bits_to_f32(((code & 0x80u) << 8) | ((code & 0x7fu) << 7)) * (sc * 256.0f);
        } else {
            const int j = c % 32;
            const uint32_t byte = row[b * 16 + (j & 15)];
            v = fp4_code(j < 16 ? byte : byte >> 4) * (sc * 16384.0f);
        }
    }
    if (use_wpe) v = v + static_cast<float>(a.wpe[(a.pos0 + t) * a.C + c]);
    static_cast<TO*>(a.out)[t * a.out_stride + c] = from_f32<TO>(v);
}

typedef void (*EmbedKernel)(EmbedArgs);

template <int FMT, typename TO>
EmbedKernel pick_wpe(bool wpe) {
    return wpe ? embed_kernel<FMT, TO, true> : embed_kernel<FMT, TO, false>;
}

template <typename TO>
EmbedKernel pick_fmt(int fmt, bool wpe) {
    switch (fmt) {
        case 0: return pick_wpe<0, TO>(wpe);
        case 1: return pick_wpe<1, TO>(wpe);
        case 2: return pick_wpe<2, TO>(wpe);
    }
    return nullptr;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_embed(neko_hip_ctx* ctx, const int32_t* tokens, int64_t T, const void* table, int64_t row_bytes,
                              int fmt, int64_t C, int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t wpe_rows,
                              int64_t pos0, void* out, int64_t out_stride, int out_dtype) {
    const char* what = "neko_hip_embed";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(out_dtype), "%s: bad dtype %d", what, out_dtype);
    NEKO_REQUIRE(ctx, fmt == NEKO_FMT_F16 || fmt == NEKO_FMT_FP8 || fmt == NEKO_FMT_FP4, "%s: bad format %d", what, fmt);
    NEKO_REQUIRE(ctx, T >= 0 && C > 0 && C <= 0x7fffffff && rows >= 0, "%s: bad shape T=%lld C=%lld rows=%lld", what,
                 (long long)T, (long long)C, (long long)rows);
    NEKO_REQUIRE(ctx, fmt == NEKO_FMT_F16 || C % 32 == 0, "%s: FP8/FP4 rows need C %% 32 == 0 (C=%lld)", what, (long long)C);
    if (T == 0 || rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, tokens && table && out, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, row_bytes >= static_cast<int64_t>(neko_quant_row_bytes(fmt, C)) && row_bytes % 2 == 0,
                 "%s: row_bytes %lld invalid for format %d and C=%lld", what, (long long)row_bytes, fmt, (long long)C);
    NEKO_REQUIRE(ctx, out_stride >= C, "%s: out stride %lld < C", what, (long long)out_stride);
    if (wpe) {
        NEKO_REQUIRE(ctx, pos0 >= 0 && pos0 + T <= wpe_rows, "%s: positions [%lld, %lld) outside the %lld-row wpe table",
                     what, (long long)pos0, (long long)(pos0 + T), (long long)wpe_rows);
    }
    const size_t osz = dtype_size(out_dtype);
    EmbedArgs a{tokens, T, static_cast<const uint8_t*>(table), row_bytes, static_cast<int>(C), row_base, rows,
                reinterpret_cast<const half_t*>(wpe), pos0, out, out_stride};
    const bool vec = (fmt != NEKO_FMT_F16 || C % 8 == 0) && aligned(table, 16) && row_bytes % 16 == 0 &&
                     aligned(out, 16) && (out_stride * osz) % 16 == 0 && (!wpe || (aligned(wpe, 16) && C % 8 == 0));
    if (vec) {
        NEKO_REQUIRE(ctx, T <= 0x7fffffffLL * 4, "%s: too many tokens", what);
        EmbedKernel k = out_dtype == NEKO_DT_F16 ? pick_fmt<half_t>(fmt, wpe != nullptr) : pick_fmt<float>(fmt, wpe != nullptr);
        hipLaunchKernelGGL(k, dim3(static_cast<uint32_t>((T + 3) / 4)), dim3(256), 0, ctx->stream, a);
        return after_launch(ctx, what);
    }
    const uint32_t gx = static_cast<uint32_t>((C + 255) / 256);
    for (int64_t t0 = 0; t0 < T; t0 += 65535) {
        EmbedArgs s = a;
        s.tokens = tokens + t0;
        s.T = T - t0 < 65535 ? T - t0 : 65535;
        s.pos0 = pos0 + t0;
        s.out = static_cast<char*>(out) + t0 * out_stride * static_cast<int64_t>(osz);
        if (out_dtype == NEKO_DT_F16)
            hipLaunchKernelGGL(embed_generic<half_t>, dim3(gx, static_cast<uint32_t>(s.T)), dim3(256), 0, ctx->stream, s, fmt,
                               wpe ? 1 : 0);
        else
            hipLaunchKernelGGL(embed_generic<float>, dim3(gx, static_cast<uint32_t>(s.T)), dim3(256), 0, ctx->stream, s, fmt,
                               wpe ? 1 : 0);
        if (int rc = after_launch(ctx, what)) return rc;
    }
    return NEKO_OK;
}
