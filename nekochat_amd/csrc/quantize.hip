// Load-time weight quantiser for gfx950: quantizeMatrix (quant.cpp:255-279) on the device, bit-identical
// to the reference's portable (x86) branch, writing the row layout the gather reads (quant.h:30-36).
//
// One thread per 32-weight block, all of a block's arithmetic in that thread in the reference's order
// (the FP4 least-squares sums are sequential float additions, so splitting a block across lanes would
// change their rounding); a wave loads its 64 blocks coalesced and hands them out through LDS.
// Divisions are IEEE (correctly rounded, hipcc's default), products are not contracted
// (-ffp-contract=off) and halfBits is one RNE f32 -> f16 conversion (subnormals kept). The FP4 fits'
// nearest-E2M1 rounding and the FP8 codes use the hardware's E2M1 / E4M3 conversions, with the
// corrections that make them equal the reference's arithmetic on every input (below). Consecutive
// threads take consecutive blocks of a row, so the code stores (16 or 32 bytes per thread) and the
// f16 scales are contiguous across the wave; the thread of a row's last block zero-fills the row's
// padding, as the reference's zero-initialised buffer leaves it.
#include <algorithm>

#include "internal.h"
#include "quant_codes.h"

namespace neko_hip {
namespace {

constexpr int kBlock = 32;  // quant.h:17 kQuantBlock

// halfBits: one RNE conversion of f as computed (f16_rne keeps a preceding multiply out of the
// conversion, so -0 products stay -0).
__device__ __forceinline__ uint32_t half_bits(float f) { return __builtin_bit_cast(uint16_t, f16_rne(f)); }
__device__ __forceinline__ float half_value(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(h)));
}

// Word w of a block's codes: byte e holds code(x[4w + e] * inv) in its low nibble and
// code(x[16 + 4w + e] * inv) in its high nibble (quant.cpp:167-178).
__device__ __forceinline__ uint32_t encode_fp4_word(const float (&x)[kBlock], int w, float inv) {
    const auto in = [&](int j) { return fp4_encode_input(x[j] * inv); };
    const int j = 4 * w;
    uint32_t word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, in(j), in(j + 16), 1.0f, 0);
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, in(j + 1), in(j + 17), 1.0f, 1);
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, in(j + 2), in(j + 18), 1.0f, 2);
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, in(j + 3), in(j + 19), 1.0f, 3);
}

struct Fit {
    float err, xr, rr;
};

// quant.cpp:126-137 (the x86 branch): sequential sums over the block.
__device__ __forceinline__ Fit fit_fp4(const float (&ax)[kBlock], float s) {
    Fit f{0.0f, 0.0f, 0.0f};
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kBlock; i += 2) {
        const float2v r = fp4_round2(ax[i] * inv, ax[i + 1] * inv);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float d = ax[i + e] - r[e] * s;
            f.err = f.err + d * d;
            f.xr = f.xr + ax[i + e] * r[e];
            f.rr = f.rr + r[e] * r[e];
        }
    }
    return f;
}

// std::max(amax, v) as the reference evaluates it: (amax < v) ? v : amax.
__device__ __forceinline__ float block_amax(const float (&x)[kBlock]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kBlock; i++) {
        const float v = fabsf(x[i]);
        amax = amax < v ? v : amax;
    }
    return amax;
}

// quant.cpp:142-165.
__device__ __forceinline__ uint32_t fp4_block_scale(const float (&x)[kBlock]) {
    const float amax = block_amax(x);
    uint32_t best = half_bits(amax / 6.0f);
    if (half_value(best) <= 0.0f) return 0;
    float ax[kBlock];
#pragma unroll
    for (int i = 0; i < kBlock; i++) ax[i] = fabsf(x[i]);
    Fit fit = fit_fp4(ax, half_value(best));
    float best_err = fit.err;
    for (int iter = 0; iter < 2 && fit.rr > 0.0f; iter++) {
        const uint32_t s = half_bits(fit.xr / fit.rr);
        if (half_value(s) <= 0.0f || s == best) break;
        fit = fit_fp4(ax, half_value(s));
        if (fit.err >= best_err) break;
        best_err = fit.err;
        best = s;
    }
    return best;
}

struct QuantArgs {
    const void* src;
    int64_t src_stride;  // elements
    uint8_t* dst;
    int64_t row_bytes;
    int64_t cols;
    int64_t pad_from;  // first padding byte of a row (codes + scales end)
    uint32_t items;    // rows * blocks per row (< 2^31)
    FastDiv nb;        // blocks per row
};

// A wave takes spans of 64 consecutive blocks. They go through LDS: the lanes load a span as
// consecutive 16-byte chunks (coalesced, whatever the row boundaries), store them with one pad word
// per 32 (block b starts at word 33 b), and each lane then reads its own block, lanes b and b+1
// landing in adjacent banks.
constexpr int kStride = kBlock + 1;

template <typename TI>
struct Span {
    static constexpr int EPC = 16 / sizeof(TI);  // elements per 16-byte chunk
    static constexpr int CPB = kBlock / EPC;     // chunks per block
    uint4v c[CPB];                               // this lane's chunks m = lane + 64 k
};

// Requests the span of blocks [block0, block0 + 64). Chunks of blocks past the last re-read the last
// block (never encoded): the loads are branch-free, so the compiler's waits for them stay partial.
template <typename TI>
__device__ __forceinline__ void load_span(const QuantArgs& a, uint32_t block0, int lane, Span<TI>& sp) {
#pragma unroll
    for (int k = 0; k < Span<TI>::CPB; k++) {
        const uint32_t m = static_cast<uint32_t>(lane) + kWave * k;
        const uint32_t blk = min(block0 + m / Span<TI>::CPB, a.items - 1);
        const uint32_t r = fast_div(blk, a.nb);
        const int64_t col = static_cast<int64_t>(blk - r * a.nb.d) * kBlock + (m % Span<TI>::CPB) * Span<TI>::EPC;
        const TI* p = static_cast<const TI*>(a.src) + static_cast<int64_t>(r) * a.src_stride + col;
        if constexpr (sizeof(TI) == 4) sp.c[k] = __builtin_bit_cast(uint4v, load_nt(reinterpret_cast<const float4v*>(p)));
        else sp.c[k] = __builtin_bit_cast(uint4v, load_nt(reinterpret_cast<const half8*>(p)));
    }
}

// Hands a loaded span out: each lane gets its own block's 32 values in x.
template <typename TI>
__device__ __forceinline__ void unstage_span(const Span<TI>& sp, float* lds, int lane, float (&x)[kBlock]) {
    // Only this wave's lanes use these words and the wave runs in lockstep, so wave-local fences (not
    // workgroup barriers) order the previous span's reads, these stores and the reads below.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < Span<TI>::CPB; k++) {
        const uint32_t m = static_cast<uint32_t>(lane) + kWave * k;
        float* d = lds + (m / Span<TI>::CPB) * kStride + (m % Span<TI>::CPB) * Span<TI>::EPC;
        if constexpr (sizeof(TI) == 4) {
            const float4v v = __builtin_bit_cast(float4v, sp.c[k]);
#pragma unroll
            for (int e = 0; e < 4; e++) d[e] = v[e];
        } else {
            const half8 v = __builtin_bit_cast(half8, sp.c[k]);
#pragma unroll
            for (int e = 0; e < 8; e++) d[e] = static_cast<float>(v[e]);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < kBlock; i++) x[i] = lds[lane * kStride + i];
}

// Block idx's codes and scale, and the row's padding from the thread of its last block.
// FMT 1: FP8 (quant.cpp:81-90), 2: FP4 (quant.cpp:167-178).
template <int FMT>
__device__ __forceinline__ void encode_block(const QuantArgs& a, uint32_t idx, const float (&x)[kBlock]) {
    const uint32_t r = fast_div(idx, a.nb);
    const uint32_t b = idx - r * a.nb.d;
    uint8_t* row = a.dst + static_cast<int64_t>(r) * a.row_bytes;
    if constexpr (FMT == 1) {
        const float amax = block_amax(x);
        const uint32_t s = half_bits(amax / 448.0f);
        const float sv = half_value(s);
        const float inv = sv > 0.0f ? 1.0f / sv : 0.0f;
        uint4v codes[2];
#pragma unroll
        for (int w = 0; w < 8; w++)
            codes[w / 4][w % 4] = encode_fp8x4(x[4 * w] * inv, x[4 * w + 1] * inv, x[4 * w + 2] * inv, x[4 * w + 3] * inv);
        uint4v* out = reinterpret_cast<uint4v*>(row + static_cast<int64_t>(b) * kBlock);
        out[0] = codes[0];
        out[1] = codes[1];
        reinterpret_cast<uint16_t*>(row + a.cols)[b] = static_cast<uint16_t>(sv > 0.0f ? s : 0u);
    } else {
        const uint32_t s = fp4_block_scale(x);
        const float inv = s ? 1.0f / half_value(s) : 0.0f;
        uint4v codes;
#pragma unroll
        for (int w = 0; w < 4; w++) codes[w] = encode_fp4_word(x, w, inv);
        *reinterpret_cast<uint4v*>(row + static_cast<int64_t>(b) * (kBlock / 2)) = codes;
        reinterpret_cast<uint16_t*>(row + a.cols / 2)[b] = static_cast<uint16_t>(s);
    }
    if (b == a.nb.d - 1)
        for (int64_t i = a.pad_from; i < a.row_bytes; i++) row[i] = 0;
}

// Persistent waves, each over spans w, w + (waves in the grid), ...: the next span's loads are in
// flight while this one is encoded. Both formats stage through LDS: with each lane loading its own
// block's 128 bytes directly, FP4 had fetched 24% extra and ran 13% slower, despite the occupancy the
// LDS costs (4 waves per SIMD).
template <int FMT, typename TI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void quantize_kernel(QuantArgs a, uint32_t spans) {
    __shared__ float lds[4][kWave * kStride];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const uint32_t step = gridDim.x * 4u;
    uint32_t sp = blockIdx.x * 4u + static_cast<uint32_t>(wave);
    if (sp >= spans) return;  // wave-uniform
    Span<TI> raw;
    load_span<TI>(a, sp * kWave, lane, raw);
    for (;;) {  // wave-uniform trip count
        float x[kBlock];
        unstage_span<TI>(raw, lds[wave], lane, x);
        const uint32_t next = sp + step;
        load_span<TI>(a, min(next, spans - 1) * kWave, lane, raw);  // past the end: re-read, unused
        const uint32_t idx = sp * kWave + static_cast<uint32_t>(lane);
        if (idx < a.items) encode_block<FMT>(a, idx, x);
        if (next >= spans) break;
        sp = next;
    }
}

// F16 rows (quant.cpp:180-186 rowToHalf): 8 elements per thread, flattened (row, chunk) space.
template <typename TI>
__global__ __launch_bounds__(256) void to_half8_kernel(const TI* src, int64_t src_stride, uint16_t* dst, int64_t cols,
                                                       uint32_t items, FastDiv cpr) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= items) return;
    const uint32_t r = fast_div(idx, cpr);
    const int64_t c = static_cast<int64_t>(idx - r * cpr.d) * 8;
    const TI* p = src + static_cast<int64_t>(r) * src_stride + c;
    half8 h;
    if constexpr (sizeof(TI) == 4) {
        const float4v lo = load_nt(reinterpret_cast<const float4v*>(p));
        const float4v hi = load_nt(reinterpret_cast<const float4v*>(p + 4));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = f16_rne(lo[e]);
            h[4 + e] = f16_rne(hi[e]);
        }
    } else {
        h = load_nt(reinterpret_cast<const half8*>(p));
    }
    *reinterpret_cast<half8*>(dst + static_cast<int64_t>(r) * cols + c) = h;
}

// Any width (the cols % 32 != 0 fallback included): one thread per element.
template <typename TI>
__global__ __launch_bounds__(256) void to_half_kernel(const TI* src, int64_t src_stride, uint16_t* dst, int64_t cols,
                                                      int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / cols, c = i - r * cols;
    dst[i] = static_cast<uint16_t>(half_bits(static_cast<float>(src[r * src_stride + c])));
}

template <typename TI>
int launch_typed(neko_hip_ctx* ctx, const char* what, int fmt, int64_t rows, int64_t cols, const void* src,
                 int64_t src_stride, uint8_t* dst, int64_t row_bytes) {
    if (fmt == NEKO_FMT_F16 && cols % 8 == 0 && aligned(src, 16) && (src_stride * sizeof(TI)) % 16 == 0 &&
        aligned(dst, 16)) {
        const int64_t cpr = cols / 8;
        const int64_t slice = 0x7fffff00LL / cpr;
        for (int64_t r0 = 0; r0 < rows; r0 += slice) {
            const int64_t n = rows - r0 < slice ? rows - r0 : slice;
            const uint32_t items = static_cast<uint32_t>(n * cpr);
            hipLaunchKernelGGL(to_half8_kernel<TI>, dim3((items + 255u) / 256u), dim3(256), 0, ctx->stream,
                               static_cast<const TI*>(src) + r0 * src_stride, src_stride,
                               reinterpret_cast<uint16_t*>(dst + r0 * row_bytes), cols, items,
                               make_fast_div(static_cast<uint32_t>(cpr)));
            if (int rc = after_launch(ctx, what)) return rc;
        }
        return NEKO_OK;
    }
    if (fmt == NEKO_FMT_F16) {
        const int64_t n = rows * cols;
        const int64_t blocks = (n + 255) / 256;
        if (blocks > 0x7fffffff) return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: too many elements", what);
        hipLaunchKernelGGL(to_half_kernel<TI>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, ctx->stream,
                           static_cast<const TI*>(src), src_stride, reinterpret_cast<uint16_t*>(dst), cols, n);
        return after_launch(ctx, what);
    }
    const int64_t nb = cols / kBlock;
    const int64_t slice = 0x7fffff00LL / nb;  // rows per launch, keeping block indices < 2^31
    for (int64_t r0 = 0; r0 < rows; r0 += slice) {
        const int64_t n = rows - r0 < slice ? rows - r0 : slice;
        QuantArgs a{static_cast<const TI*>(src) + r0 * src_stride, src_stride, dst + r0 * row_bytes, row_bytes, cols,
                    fmt == NEKO_FMT_FP8 ? cols + 2 * nb : cols / 2 + 2 * nb, static_cast<uint32_t>(n * nb),
                    make_fast_div(static_cast<uint32_t>(nb))};
        if (a.items == 0) continue;
        // One workgroup per LDS slot of the chip (four fit a CU), each wave looping over spans.
        const uint32_t spans = (a.items + kWave - 1) / kWave;
        const uint32_t blocks = std::min<uint32_t>((spans + 3u) / 4u, static_cast<uint32_t>(4 * std::max(1, ctx->cu_count)));
        if (fmt == NEKO_FMT_FP8)
            hipLaunchKernelGGL((quantize_kernel<1, TI>), dim3(blocks), dim3(256), 0, ctx->stream, a, spans);
        else
            hipLaunchKernelGGL((quantize_kernel<2, TI>), dim3(blocks), dim3(256), 0, ctx->stream, a, spans);
        if (int rc = after_launch(ctx, what)) return rc;
    }
    return NEKO_OK;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_quantize_rows(neko_hip_ctx* ctx, int fmt, int64_t rows, int64_t cols, const void* src,
                                      int64_t src_stride, int src_dtype, uint8_t* dst, int* fmt_used) {
    const char* what = "neko_hip_quantize_rows";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, fmt == NEKO_FMT_F16 || fmt == NEKO_FMT_FP8 || fmt == NEKO_FMT_FP4, "%s: bad format %d", what, fmt);
    NEKO_REQUIRE(ctx, valid_dtype(src_dtype), "%s: bad source dtype %d", what, src_dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && cols > 0 && cols <= 0x7fffffff, "%s: bad shape rows=%lld cols=%lld", what,
                 (long long)rows, (long long)cols);
    const int used = cols % kBlock != 0 ? NEKO_FMT_F16 : fmt;  // quant.cpp:257
    if (fmt_used) *fmt_used = used;
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, src && dst, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, src_stride >= cols, "%s: source stride %lld < cols %lld", what, (long long)src_stride, (long long)cols);
    const int64_t row_bytes = static_cast<int64_t>(neko_quant_row_bytes(used, cols));
    if (used != NEKO_FMT_F16) {
        const size_t esz = dtype_size(src_dtype);
        NEKO_REQUIRE(ctx, aligned(src, 16) && (src_stride * esz) % 16 == 0 && aligned(dst, 16),
                     "%s: FP8/FP4 need 16-byte aligned source rows and output", what);
    }
    return src_dtype == NEKO_DT_F32 ? launch_typed<float>(ctx, what, used, rows, cols, src, src_stride, dst, row_bytes)
                                    : launch_typed<half_t>(ctx, what, used, rows, cols, src, src_stride, dst, row_bytes);
}
