// Embedding gather with fused row dequantisation for gfx950 (embed.comp:1-51,
// QMatrix::dequantizeRow quant.cpp:230-253, GPT-2 wte + wpe gpt2_model.cpp:182-187).
//
// Each wavefront gathers a few consecutive tokens with all their rows' loads in flight at once; each
// lane produces one 16-byte chunk of an output row per step (see embed_kernel), so every store
// instruction writes whole cache lines.
// Codes are decoded with the reference's bit trick (the code's bits placed into an f16 pattern that
// equals value / 256 for E4M3 or value / 16384 for E2M1, subnormals included), then multiplied in
// f32 by scale * 256 (or * 16384). Every such product has at most 15 significant bits, so it is
// exact and identical to the reference's f32 value; f16 output is one RNE rounding of it (or, for
// f16 output without wpe, the same rounding done by a packed f16 multiply, see fp8_pair_bits). This
// keeps the reference's 0x7F / 0xFF = +-480 (not NaN) and -0 codes. With wpe the position row is
// added in f32 first, then rounded once, as the reference does.
#include <type_traits>

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
    float scale;  // the rows' f32 multiplier (Granite's embedding_multiplier; 1 for plain gathers)
};

// What the gather adds to the dequantised row: nothing, GPT-2's position row (added in f32), or a
// multiplier (granite_model.cpp:298-301: x[c] *= embeddingMult, one f32 rounding).
enum class Extra : int { None = 0, Wpe = 1, Scale = 2 };

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

// Packed-f16 decoding, for f16 output without a position table: two codes (in the low bits of the
// two 16-bit halves of p) become the f16 patterns above, which one v_pk_mul_f16 by 2^8 (FP8) or
// 2^14 (FP4) turns exactly into the code values and a second multiplies by the f16 block scale. The
// product of two f16 values is exact in f32, so the single RNE rounding of the f16 multiply equals
// the reference's f32 product rounded to f16 (f16 subnormals are kept, as the hardware does by
// default for f16).
// (fp8_pair_bits / fp4_pair_bits, device.h)

// 32-bit word w of a loaded chunk (a scalar when the chunk is one word).
template <typename R>
__device__ __forceinline__ uint32_t word_of(const R& r, int w) {
    if constexpr (sizeof(R) == 4) return static_cast<uint32_t>(r);
    else return static_cast<uint32_t>(r[w]);
}

// Launch shape (the fastest measured on MI355X for a 16384-token gather of 2048-wide rows): four
// tokens per wavefront for every format (two: F16 20.8, FP8 18.5, FP4 17.5 us against 19.0 / 17.5 /
// 15.4 with four) and four 16-byte output chunks per lane per token in flight.
__host__ __device__ constexpr int chunks_in_flight(int) { return 4; }
__host__ __device__ constexpr int tokens_per_wave(int) { return 4; }

// Vector path. FMT: 0 F16, 1 FP8, 2 FP4. The output row is cut into chunks of EPC = 16 bytes of
// output elements (8 halves or 4 floats); lane l takes chunks l, l + 64, ..., so every store
// instruction writes 1 KB of contiguous output (whole cache lines). Each chunk loads exactly the
// stored bytes it decodes: EPC halves (F16), EPC code bytes (FP8), or the EPC bytes of its 32-weight
// block that hold its elements (FP4: elements j < 16 sit in the low nibbles of bytes j, elements
// 16 + j in the high nibbles). Requires C % 32 == 0 for FP8/FP4, C % EPC == 0 for F16, and
// 16-byte aligned output rows (plus 2 * EPC-byte aligned table rows and wpe rows).
// FP4 with f16 output: the four lanes of a quad hold the four chunks of one 32-weight block (chunk c
// of lane l has c % 4 == l % 4), whose 16 code bytes each chunk needs half of: each lane loads one
// dword of the block and takes the two it decodes from its quad by DPP, so the row's code bytes are
// loaded once (measured for a 16384-token Zipf gather of 2048-wide rows: 16.8 us against 19.7 for
// 8-byte loads per chunk, which fetch every byte twice).
// Each wave owns tokens_per_wave(FMT) consecutive tokens: their ids come in one load, then every
// row's chunk loads are issued before any is decoded. Two ways to move the bytes, chosen per format
// by measurement (16384 Zipf tokens of 2048-wide rows, f16 out, side by side):
// - F16 and FP8: plain loads and stores per chunk (a chunk past the row's end skips both), FP8's block
//   scale loaded per chunk: 19.0 / 17.5 us, on the floors of their patterns (19.0 / 17.2); the form
//   below took 20.3 / 19.2.
// - FP4: every load and store through range-checked buffer resources (device.h), so nothing is under a
//   branch and the compiler's memory-counter waits stay per token, and one dword of block scales per
//   lane and step shared by ds_bpermute: 15.4 us, under its floor (16.1); the form above took 16.5.
template <int FMT, typename TO, Extra X>
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
    constexpr bool WPE = X == Extra::Wpe;
    constexpr bool kRes = FMT == 2;
    constexpr int EPC = 16 / sizeof(TO);  // output elements per chunk
    constexpr int TPW = tokens_per_wave(FMT);  // tokens per wave, all in flight together
    constexpr int B = chunks_in_flight(FMT);   // chunks per lane per token in flight
    typedef typename VecOf<TO, EPC>::V VO;
    typedef typename VecOf<half_t, EPC>::V VH;
    // FP8 / FP4 decoded in packed f16 when the output is f16 and nothing is added or multiplied.
    constexpr bool kPacked = FMT != 0 && EPC == 8 && X == Extra::None;
    // Raw chunk bytes: F16 2*EPC bytes, FP8/FP4 EPC bytes (FP4 with f16 output: one dword of the block,
    // the quad's shared load).
    constexpr bool kQuad = FMT == 2 && EPC == 8;
    typedef typename VecOf<uint32_t, (FMT == 0 ? 2 * EPC : EPC) / 4>::V Raw;
    typedef typename std::conditional<kQuad, uint32_t, Raw>::type Load;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * TPW;
    if (t0 >= a.T) return;
    // The wave's token ids in one load (lane i holds token t0 + i), then broadcast as scalars.
    const int32_t my_id = lane < TPW && t0 + lane < a.T ? a.tokens[t0 + lane] : 0;
    // Each token's row: a pointer, and for kRes a resource over it (empty for a token outside this table
    // chunk; loads past a resource return zeros with no memory access, stores past it are dropped).
    const uint8_t* rowp[TPW];
    BufRes rowr[TPW], wper[TPW];
    bool live[TPW];
    const uint32_t rbytes = static_cast<uint32_t>(a.row_bytes);
#pragma unroll
    for (int k = 0; k < TPW; k++) {
        const int64_t r = static_cast<int64_t>(__builtin_amdgcn_readlane(my_id, k)) - a.row_base;
        live[k] = t0 + k < a.T && r >= 0 && r < a.rows;  // other tokens belong to another table chunk
        rowp[k] = a.table + (live[k] ? r : 0) * a.row_bytes;
        if constexpr (kRes) {
            rowr[k] = buf_res(rowp[k], live[k] ? rbytes : 0u);
            if constexpr (WPE)
                wper[k] = buf_res(a.wpe + (live[k] ? a.pos0 + t0 + k : 0) * a.C, live[k] ? static_cast<uint32_t>(a.C) * 2u : 0u);
        }
    }
    const int nch = a.C / EPC;
    const int64_t soff = FMT == 1 ? a.C : a.C / 2;  // scales follow the codes
    // kRes block scales: a step of B * 64 chunks spans (B * 64) / CPB blocks (at most 64 halves: 32
    // dwords); lane l loads dword l % 32 of them and each lane takes its chunk's scale from the lane
    // holding it (ds_bpermute).
    constexpr int CPB = 32 / EPC;  // chunks per 32-wide block
    static_assert(B * kWave / CPB <= 64, "one dword of scales per lane covers a step");

    for (int c0 = 0; c0 < nch; c0 += B * kWave) {
        Load raw[TPW][B];
        half_t sc[TPW][B];
        uint32_t scw[TPW];
        VH pw[TPW][B];
        const uint32_t blk0 = static_cast<uint32_t>(c0 / CPB);  // the step's first block (c0: a multiple of B * 64)
#pragma unroll
        for (int k = 0; k < TPW; k++) {
            if constexpr (kRes) {
                scw[k] = buf_load<uint32_t>(rowr[k], static_cast<uint32_t>(soff) + 2 * blk0 + 4 * (lane & 31));
#pragma unroll
                for (int b = 0; b < B; b++) {
                    // Chunks past the row's last one load whatever the row holds there, or zeros past
                    // its end; they are not stored.
                    const uint32_t e0 = static_cast<uint32_t>((c0 + b * kWave + lane) * EPC);
                    const uint32_t blk = e0 >> 5, j0 = e0 & 15;
                    if constexpr (kQuad) raw[k][b] = buf_load<uint32_t>(rowr[k], 16 * blk + 4 * (lane & 3));
                    else raw[k][b] = buf_load<Raw>(rowr[k], 16 * blk + j0);
                    if constexpr (WPE) pw[k][b] = buf_load<VH>(wper[k], 2 * e0);
                }
            } else {
                if (!live[k]) continue;
                const uint8_t* row = rowp[k];
#pragma unroll
                for (int b = 0; b < B; b++) {
                    const int c = c0 + b * kWave + lane;
                    if (c >= nch) continue;
                    const int e0 = c * EPC;
                    if constexpr (FMT == 0) {
                        raw[k][b] = *reinterpret_cast<const Raw*>(row + 2 * e0);
                    } else {
                        raw[k][b] = *reinterpret_cast<const Raw*>(row + e0);
                        sc[k][b] = *reinterpret_cast<const half_t*>(row + soff + 2 * (e0 >> 5));
                    }
                    if constexpr (WPE) pw[k][b] = *reinterpret_cast<const VH*>(a.wpe + (a.pos0 + t0 + k) * a.C + e0);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < TPW; k++) {
            if constexpr (!kRes) {
                if (!live[k]) continue;
            }
            TO* out = static_cast<TO*>(a.out) + (t0 + k) * a.out_stride;
            const BufRes outr = buf_res(out, kRes && live[k] ? static_cast<uint32_t>(a.C * sizeof(TO)) : 0u);
            // kRes: each chunk's block scale from the lane that loaded it (all lanes active here).
            half_t scs[B];
            if constexpr (kRes) {
#pragma unroll
                for (int b = 0; b < B; b++) {
                    const int rb = (b * kWave + lane) / CPB;  // block relative to blk0
                    const half2v s2 = __builtin_bit_cast(
                        half2v, __builtin_amdgcn_ds_bpermute(4 * (rb >> 1), static_cast<int>(scw[k])));
                    scs[b] = s2[rb & 1];
                }
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int c = c0 + b * kWave + lane;
                if constexpr (!kRes) {
                    if (c >= nch) continue;
                    if constexpr (FMT != 0) scs[b] = sc[k][b];
                }
                // The chunk's code bytes: FP4 quad loads give lane q of a quad the block's bytes 0-7
                // (q = 0, 2) or 8-15 (q = 1, 3), the dwords of quad lanes 2 (q % 2) and 2 (q % 2) + 1.
                Raw rw;
                if constexpr (kQuad) {
                    const int d = static_cast<int>(raw[k][b]);
                    rw[0] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, d, kDppQuadPairLo, 0xF, 0xF, false));
                    rw[1] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, d, kDppQuadPairHi, 0xF, 0xF, false));
                } else {
                    rw = raw[k][b];
                }
                VO o;
                if constexpr (kPacked) {
                    const half2v s2 = {scs[b], scs[b]};
                    const half2v k2 = FMT == 1 ? half2v{256.0f16, 256.0f16} : half2v{16384.0f16, 16384.0f16};
                    const int shift = FMT == 2 && ((c * EPC) & 16) ? 4 : 0;
                    uint4v ob;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t word = word_of(rw, i >> 1) >> shift;
                        const uint32_t p = __builtin_amdgcn_perm(0u, word, (i & 1) ? 0x0C030C02u : 0x0C010C00u);
                        const uint32_t bits = FMT == 1 ? fp8_pair_bits(p) : fp4_pair_bits(p);
                        ob[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, bits) * k2 * s2);
                    }
                    o = __builtin_bit_cast(VO, ob);
                } else {
                    float v[EPC];
                    if constexpr (FMT == 0) {
                        const VH h = __builtin_bit_cast(VH, rw);
#pragma unroll
                        for (int e = 0; e < EPC; e++) v[e] = static_cast<float>(h[e]);
                    } else if constexpr (FMT == 1) {
                        const float sf = static_cast<float>(scs[b]) * 256.0f;
#pragma unroll
                        for (int w = 0; w < EPC / 4; w++) {
                            const uint32_t word = word_of(rw, w);
                            float f0, f1, f2, f3;
                            fp8_pair(word, f0, f1);
                            fp8_pair(word >> 16, f2, f3);
                            v[4 * w + 0] = f0 * sf;
                            v[4 * w + 1] = f1 * sf;
                            v[4 * w + 2] = f2 * sf;
                            v[4 * w + 3] = f3 * sf;
                        }
                    } else {
                        const int shift = ((c * EPC) & 16) ? 4 : 0;  // high nibbles for elements 16..31 of the block
                        const float sf = static_cast<float>(scs[b]) * 16384.0f;
#pragma unroll
                        for (int w = 0; w < EPC / 4; w++) {
                            const uint32_t word = word_of(rw, w) >> shift;
#pragma unroll
                            for (int q = 0; q < 4; q++) v[4 * w + q] = fp4_code(word >> (8 * q)) * sf;
                        }
                    }
                    if constexpr (WPE) {
#pragma unroll
                        for (int e = 0; e < EPC; e++) v[e] = v[e] + static_cast<float>(pw[k][b][e]);
                    }
                    if constexpr (X == Extra::Scale) {
#pragma unroll
                        for (int e = 0; e < EPC; e++) v[e] = v[e] * a.scale;
                    }
#pragma unroll
                    for (int e = 0; e < EPC; e++) o[e] = from_f32<TO>(v[e]);
                }
                // plain stores (non-temporal ones were no faster)
                if constexpr (kRes) buf_store16<false>(outr, static_cast<uint32_t>(c) * 16u, o);
                else *reinterpret_cast<VO*>(out + c * EPC) = o;
            }
        }
    }
}

// Any layout: one thread per element, byte addressing (the embed.comp scheme).
template <typename TO>
__global__ __launch_bounds__(256) void embed_generic(EmbedArgs a, int fmt, int use_wpe, int use_scale) {
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
    if (use_scale) v = v * a.scale;
    static_cast<TO*>(a.out)[t * a.out_stride + c] = from_f32<TO>(v);
}

typedef void (*EmbedKernel)(EmbedArgs);

template <int FMT, typename TO>
EmbedKernel pick_extra(Extra x) {
    return x == Extra::Wpe     ? embed_kernel<FMT, TO, Extra::Wpe>
           : x == Extra::Scale ? embed_kernel<FMT, TO, Extra::Scale>
                               : embed_kernel<FMT, TO, Extra::None>;
}

template <typename TO>
EmbedKernel pick_fmt(int fmt, Extra x) {
    switch (fmt) {
        case 0: return pick_extra<0, TO>(x);
        case 1: return pick_extra<1, TO>(x);
        case 2: return pick_extra<2, TO>(x);
    }
    return nullptr;
}

// Argument checks, then the vector kernel or (any layout) the per-element one.
int launch_embed(neko_hip_ctx* ctx, const char* what, const int32_t* tokens, int64_t T, const void* table, int64_t row_bytes,
                 int fmt, int64_t C, int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t wpe_rows, int64_t pos0,
                 float scale, bool scaled, void* out, int64_t out_stride, int out_dtype) {
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
    const Extra extra = wpe ? Extra::Wpe : scaled ? Extra::Scale : Extra::None;
    const size_t osz = dtype_size(out_dtype);
    EmbedArgs a{tokens, T, static_cast<const uint8_t*>(table), row_bytes, static_cast<int>(C), row_base, rows,
                reinterpret_cast<const half_t*>(wpe), pos0, out, out_stride, scale};
    // Chunks of 16 output bytes: EPC elements; loads of 2*EPC (F16) or EPC (FP8/FP4) table bytes.
    const int64_t epc = static_cast<int64_t>(16 / osz);
    const int64_t chunk_in = fmt == NEKO_FMT_F16 ? 2 * epc : epc;
    const bool vec = C % epc == 0 && aligned(table, static_cast<size_t>(chunk_in)) && row_bytes % chunk_in == 0 &&
                     aligned(out, 16) && (out_stride * osz) % 16 == 0 &&
                     (!wpe || (aligned(wpe, static_cast<size_t>(2 * epc)) && (C * 2) % (2 * epc) == 0));
    if (vec) {
        const int64_t per_block = 4 * tokens_per_wave(fmt);
        NEKO_REQUIRE(ctx, T <= 0x7fffffffLL * per_block, "%s: too many tokens", what);
        EmbedKernel k = out_dtype == NEKO_DT_F16 ? pick_fmt<half_t>(fmt, extra) : pick_fmt<float>(fmt, extra);
        hipLaunchKernelGGL(k, dim3(static_cast<uint32_t>((T + per_block - 1) / per_block)), dim3(256), 0, ctx->stream, a);
        return after_launch(ctx, what);
    }
    const uint32_t gx = static_cast<uint32_t>((C + 255) / 256);
    for (int64_t t0 = 0; t0 < T; t0 += 65535) {
        EmbedArgs s = a;
        s.tokens = tokens + t0;
        s.T = T - t0 < 65535 ? T - t0 : 65535;
        s.pos0 = pos0 + t0;
        s.out = static_cast<char*>(out) + t0 * out_stride * static_cast<int64_t>(osz);
        const int w = wpe ? 1 : 0, sc = scaled ? 1 : 0;
        if (out_dtype == NEKO_DT_F16)
            hipLaunchKernelGGL(embed_generic<half_t>, dim3(gx, static_cast<uint32_t>(s.T)), dim3(256), 0, ctx->stream, s, fmt,
                               w, sc);
        else
            hipLaunchKernelGGL(embed_generic<float>, dim3(gx, static_cast<uint32_t>(s.T)), dim3(256), 0, ctx->stream, s, fmt,
                               w, sc);
        if (int rc = after_launch(ctx, what)) return rc;
    }
    return NEKO_OK;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_embed(neko_hip_ctx* ctx, const int32_t* tokens, int64_t T, const void* table, int64_t row_bytes,
                              int fmt, int64_t C, int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t wpe_rows,
                              int64_t pos0, void* out, int64_t out_stride, int out_dtype) {
    return launch_embed(ctx, "neko_hip_embed", tokens, T, table, row_bytes, fmt, C, row_base, rows, wpe, wpe_rows, pos0,
                        1.0f, false, out, out_stride, out_dtype);
}

extern "C" int neko_hip_embed_scaled(neko_hip_ctx* ctx, const int32_t* tokens, int64_t T, const void* table,
                                     int64_t row_bytes, int fmt, int64_t C, int64_t row_base, int64_t rows, float scale,
                                     void* out, int64_t out_stride, int out_dtype) {
    return launch_embed(ctx, "neko_hip_embed_scaled", tokens, T, table, row_bytes, fmt, C, row_base, rows, nullptr, 0, 0,
                        scale, true, out, out_stride, out_dtype);
}
