// Weight matmul for gfx950: y[t][n] (+)= act(x[t] . W[n] + bias[n]) with W stored in the reference's
// weight row formats -- F16, FP8 (E4M3 codes + f16 block scales) and FP4 (E2M1 nibbles + f16 block
// scales), quant.h:30-36. The reference's Matmul / MatmulQ8 / MatmulQ4 kernels (matmul.comp,
// matmul_q8.comp, matmul_q4.comp) and cpu::matmul (cpu_ops.cpp:474-490).
//
// Fast path (f16 activations, K % 32 == 0): one wave owns a tile of 16 weight rows and up to 64
// tokens and walks a slice of K in 32-wide blocks -- exactly one FP8/FP4 scale block -- with
// v_mfma_f32_16x16x32_f16. The weight codes enter the MFMA as the exact f16 values code/2^8 (FP8) or
// code/2^14 (FP4), the activations as they are, so every product is exact and summed in f32; the
// block's f32 sum is then multiplied by its f16 scale (times 2^8 or 2^14, exact) and accumulated
// with one fma. F16 rows feed the MFMA directly. The workgroup's waves split K and add their
// partial tiles in LDS in a fixed order, then apply bias, GELU and the accumulate epilogue. Rows
// are read once per 64 tokens, so for decode-sized T the kernel is a stream of the weight bytes.
//
// Generic path (f32 activations, unaligned or odd shapes): one wave per weight row and 4 tokens,
// lanes striding K, each weight decoded exactly to f32 and multiplied and added in f32.
//
// Summation order differs from the reference's sequential dot (and the reference's own GPU shaders
// differ from its CPU loop), so results agree to f32 rounding of the sum, not bit for bit.
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>

#include "internal.h"

namespace neko_hip {
namespace {

constexpr int kBlockK = 32;  // quant.h kQuantBlock

// Kernels taking more than 64 KB of dynamic LDS must be allowed it per device (hipFuncSetAttribute on
// the context's device, which enter() made current); `done` records which devices have been, one bit
// per device id, safely across host threads.
int allow_lds(neko_hip_ctx* ctx, const void* kernel, size_t bytes, std::atomic<uint64_t>& done) {
    const uint64_t bit = uint64_t(1) << (ctx->device & 63);
    if (done.load(std::memory_order_acquire) & bit) return NEKO_OK;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return fail(ctx, NEKO_ERR_HIP, "matmul: hipFuncSetAttribute: %s", hipGetErrorString(e));
    done.fetch_or(bit, std::memory_order_release);
    return NEKO_OK;
}

struct MmArgs {
    const void* x;
    int64_t xs;
    int64_t T;
    const uint8_t* w;
    int64_t rb;
    int K;
    int N;
    const float* bias;
    void* y;
    int64_t ys;
    int flags;
    int fmt;
    int blocks_per_wave;  // 32-wide blocks of K per wave, a multiple of kGroup (fast path)
    int vec_y;            // 1: every run of 4 outputs starting at a multiple of 4 is naturally aligned
};

constexpr int kGelu = 1, kAccumulate = 2;  // cpu_ops.h MatmulFlags

template <typename TY>
__device__ __forceinline__ void epilogue(const MmArgs& a, int64_t t, int64_t n, float v) {
    if (a.bias) v += a.bias[n];
    if (a.flags & kGelu) v = gelu_ref(v);
    TY* yp = static_cast<TY*>(a.y) + t * a.ys + n;
    if (a.flags & kAccumulate) v += to_f32(*yp);
    *yp = from_f32<TY>(v);
}

// LDS floats a wave needs to regroup one 32 x 32 accumulator tile (rows padded to 36 floats: 16-byte
// aligned, and the two row groups one write instruction covers fall on different banks).
constexpr int kTileLdsRow = 36;
constexpr int kTileLdsFloats = 32 * kTileLdsRow;

// Outputs n .. n + 3 of row t from a regrouped tile row in LDS (`src` holds their four values), GELU
// applied or not at compile time: one 4-element load and store when all four exist and a.vec_y says
// they are aligned, else element by element in a loop that stays rolled (the rare tail / unaligned
// case; rereading LDS keeps it one copy). Rows t >= T are skipped.
template <typename TY, bool GELU>
__device__ __forceinline__ void epilogue4_lds(const MmArgs& a, int64_t t, int64_t n, const float* src) {
    if (t >= a.T) return;
    if (a.vec_y && n + 4 <= a.N) {
        typedef typename VecOf<TY, 4>::V V4;
        float4v v = *reinterpret_cast<const float4v*>(src);
        if (a.bias) {
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] += a.bias[n + q];
        }
        if constexpr (GELU) {
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = gelu_ref(v[q]);
        }
        V4* yp = reinterpret_cast<V4*>(static_cast<TY*>(a.y) + t * a.ys + n);
        if (a.flags & kAccumulate) {
            const V4 old = *yp;
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] += to_f32(old[q]);
        }
        V4 o;
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = from_f32<TY>(v[q]);
        *yp = o;
    } else {
#pragma unroll 1
        for (int q = 0; q < 4 && n + q < a.N; q++) {
            float v = src[q];
            if (a.bias) v += a.bias[n + q];
            if constexpr (GELU) v = gelu_ref(v);
            TY* yp = static_cast<TY*>(a.y) + t * a.ys + n + q;
            if (a.flags & kAccumulate) v += to_f32(*yp);
            *yp = from_f32<TY>(v);
        }
    }
}

template <typename TY, int TM, int TN, bool GELU>
__device__ __forceinline__ void store_tiles_as(const MmArgs& a, const float16v (&acc)[TM][TN], float* scratch, int64_t m_base,
                                               int64_t n_base, int lane) {
    const int l32 = lane & 31, h = lane >> 5;
    const int rr = lane >> 3, cc = 4 * (lane & 7);
    unrolled<TM>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        unrolled<TN>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float16v v = acc[i][j];
            unrolled<16>([&](auto ec) {
                constexpr int e = decltype(ec)::value;
                scratch[(8 * (e >> 2) + 4 * h + (e & 3)) * kTileLdsRow + l32] = v[e];
            });
            if constexpr (GELU) {
#pragma unroll 1
                for (int r = 0; r < 4; r++) {
                    const int row = 8 * r + rr;
                    epilogue4_lds<TY, true>(a, m_base + i * 32 + row, n_base + j * 32 + cc, &scratch[row * kTileLdsRow + cc]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = 8 * r + rr;
                    epilogue4_lds<TY, false>(a, m_base + i * 32 + row, n_base + j * 32 + cc, &scratch[row * kTileLdsRow + cc]);
                }
            }
        });
    });
}

// Stores a wave's TM x TN grid of 32 x 32 v_mfma_f32_32x32x16 accumulator tiles -- lane (l32, h) holds
// C[8 (e / 4) + 4 h + e % 4][l32] of each -- as 4-output row chunks: each tile is written to the
// wave's LDS scratch (kTileLdsFloats) and read back so that lane l takes columns 4 (l % 8) .. + 3 of
// rows l / 8, 8 + l / 8, ...; every store instruction then covers eight whole 128-byte row segments,
// with a quarter of the instructions of element-wise stores. Tile (i, j) covers rows m_base + 32 i ..
// and columns n_base + 32 j ... The GELU epilogue is a separate instantiation chosen once per call:
// inlined into every tile's rows it made the kernel's code several hundred KB, which the instruction
// cache then streamed through on every tile's epilogue.
template <typename TY, int TM, int TN>
__device__ __forceinline__ void store_tiles(const MmArgs& a, const float16v (&acc)[TM][TN], float* scratch, int64_t m_base,
                                            int64_t n_base, int lane) {
    if (a.flags & kGelu) store_tiles_as<TY, TM, TN, true>(a, acc, scratch, m_base, n_base, lane);
    else store_tiles_as<TY, TM, TN, false>(a, acc, scratch, m_base, n_base, lane);
}

// ---------------------------------------------------------------- fast path: MFMA tiles

// The B operand of one 32-wide block for weight row `row`: the 8 k values lane group g supplies.
// FP8: codes g*8 .. g*8+7 of the block (8 bytes). FP4: bytes g*4 .. g*4+3 of the 16-byte block, low
// nibbles (k = g*4 + i) then high nibbles (k = 16 + g*4 + i). F16: halves g*8 .. g*8+7. Loaded raw
// (so a group can be fetched ahead) and decoded to exact f16 values just before its MFMA.

template <int FMT>
struct BRaw {
    typedef half8 T;
};
template <>
struct BRaw<1> {
    typedef uint2v T;
};
template <>
struct BRaw<2> {
    typedef uint32_t T;
};

template <int FMT>
__device__ __forceinline__ typename BRaw<FMT>::T load_b_raw(const uint8_t* row, int b, int g) {
    if constexpr (FMT == 0) return *reinterpret_cast<const half8*>(row + 2 * (b * kBlockK + g * 8));
    else if constexpr (FMT == 1) return *reinterpret_cast<const uint2v*>(row + b * kBlockK + g * 8);
    else return *reinterpret_cast<const uint32_t*>(row + b * (kBlockK / 2) + g * 4);
}

template <int FMT>
__device__ __forceinline__ half8 decode_b(typename BRaw<FMT>::T q) {
    if constexpr (FMT == 0) {
        return q;
    } else if constexpr (FMT == 1) {
        uint4v h;
        h[0] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q[0], 0x0C010C00u));
        h[1] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q[0], 0x0C030C02u));
        h[2] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q[1], 0x0C010C00u));
        h[3] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q[1], 0x0C030C02u));
        return __builtin_bit_cast(half8, h);
    } else {
        // gfx950's E2M1 -> f16 conversion (scale 1: the code values themselves, exact, -0 for code 8):
        // byte i -> [low nibble, high nibble]; regrouped into the low nibbles of bytes 0..3 then the
        // high nibbles.
        const uint32_t c[4] = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 1.0f, 0)),
                               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 1.0f, 1)),
                               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 1.0f, 2)),
                               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q, 1.0f, 3))};
        uint4v h;
        h[0] = __builtin_amdgcn_perm(c[1], c[0], 0x05040100u);
        h[1] = __builtin_amdgcn_perm(c[3], c[2], 0x05040100u);
        h[2] = __builtin_amdgcn_perm(c[1], c[0], 0x07060302u);
        h[3] = __builtin_amdgcn_perm(c[3], c[2], 0x07060302u);
        return __builtin_bit_cast(half8, h);
    }
}

// The matching A operand: activations of one token at the same 8 k positions.
template <int FMT>
__device__ __forceinline__ half8 load_a(const half_t* xr, int b, int g) {
    if constexpr (FMT == 2) {
        const uint2v lo = *reinterpret_cast<const uint2v*>(xr + b * kBlockK + g * 4);
        const uint2v hi = *reinterpret_cast<const uint2v*>(xr + b * kBlockK + 16 + g * 4);
        return __builtin_bit_cast(half8, uint4v{lo[0], lo[1], hi[0], hi[1]});
    } else {
        return *reinterpret_cast<const half8*>(xr + b * kBlockK + g * 8);
    }
}

// What the block sum is multiplied by besides the f16 scale: decoded FP8 codes are value / 2^8; FP4
// codes, from the hardware conversion, the values themselves.
template <int FMT>
__device__ __forceinline__ float block_scale_factor() {
    return FMT == 1 ? 256.0f : 1.0f;
}

// One 32-wide block: acc[tt] += scale * (x-tile . codes) (FP8/FP4) or acc[tt] += x-tile . w (F16).
template <int FMT, int TT>
__device__ __forceinline__ void mma_block(float4v (&acc)[TT], const half8 (&A)[TT], half8 B, float s) {
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        if constexpr (FMT == 0) {
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[tt], B, acc[tt], 0, 0, 0);
        } else {
            const float4v blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[tt], B, float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[tt][i] = __builtin_fmaf(s, blk[i], acc[tt][i]);
        }
    }
}

// Weights travel in groups of four 32-wide blocks of each of the tile's 16 rows (256 / 128 / 64
// contiguous bytes per row for F16 / FP8 / FP4): lanes load a group coalesced, 16 bytes each along
// the rows, write it to the wave's LDS tile and read their MFMA operands back from there -- a direct
// MFMA-layout load would touch 16 rows per instruction for 4-16 bytes of each. Launch shape: waves per
// row tile (the K split) chosen for about kWaveTarget waves in the grid, at most kMaxWaves per
// workgroup (1024 measured 3-9% faster than 2048-16384 over the Qwen3-4B projections at 3-8 tokens:
// fewer waves per tile, less cross-wave reduction).
constexpr int64_t kWaveTarget = 1024;
constexpr int kMaxWaves = 16;
constexpr int kGroup = 4;  // 32-wide blocks per group: one 8-byte load of a row's 4 block scales

// Bytes of one row's 32-wide block; a group's bytes of one row; 16-byte pieces per lane per group.
__host__ __device__ constexpr int block_bytes(int fmt) { return fmt == 0 ? 64 : fmt == 1 ? 32 : 16; }
__host__ __device__ constexpr int group_row_bytes(int fmt) { return kGroup * block_bytes(fmt); }
__host__ __device__ constexpr int pieces(int fmt) { return group_row_bytes(fmt) / 64; }  // 16 rows / 64 lanes / 16 B
__host__ __device__ constexpr int stage_row(int fmt) { return group_row_bytes(fmt) + 16; }  // padded: no bank conflicts
__host__ __device__ constexpr int stage_bytes(int fmt) { return 16 * stage_row(fmt); }      // one wave's tile

template <int FMT>
struct MmStage {
    uint4v w[pieces(FMT)];  // this lane's 16-byte pieces of the group
    uint2v s;               // this lane's row's 4 block scales (FP8 / FP4)
};

// Requests group b0's weight pieces and scales. Piece i of lane l is chunk c = 64 i + l of the
// group: row c / (pieces per row), 16-byte column c % (pieces per row); rows[i] are those rows.
template <int FMT>
__device__ __forceinline__ void load_stage(MmStage<FMT>& st, const uint8_t* const (&rows)[pieces(FMT)], int col16,
                                           const uint8_t* wrow, int soff, int b0) {
#pragma unroll
    for (int i = 0; i < pieces(FMT); i++)
        st.w[i] = *reinterpret_cast<const uint4v*>(rows[i] + b0 * block_bytes(FMT) + col16 * 16);
    if constexpr (FMT != 0) st.s = *reinterpret_cast<const uint2v*>(wrow + soff + 2 * b0);
}

// Activations of a group. Every lane loads, without a branch: a lane whose token row is past T
// reads row 0 (a valid address) and feeds it to MFMA output rows that are never stored (each
// output row depends only on its own A row). Loads under divergent control flow, or values used
// at once, would make the compiler wait for every outstanding load and drain the weight prefetch.
template <int FMT, int TT>
__device__ __forceinline__ void load_acts(half8 (&A)[kGroup][TT], const half_t* const (&xr)[TT], int b0, int g) {
#pragma unroll
    for (int j = 0; j < kGroup; j++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) A[j][tt] = load_a<FMT>(xr[tt], b0 + j, g);
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int FMT>
__device__ __forceinline__ typename BRaw<FMT>::T read_b(const uint8_t* tile, int n, int j, int g) {
    const uint8_t* p = tile + n * stage_row(FMT) + j * block_bytes(FMT) + g * (block_bytes(FMT) / 4);
    return *reinterpret_cast<const typename BRaw<FMT>::T*>(p);
}

// One group: request the next group's activations, write this group's weights to the wave's LDS
// tile, request the weights two groups ahead into the same registers, then the group's MFMAs.
// (hipcc keeps `sc` in the old scale registers and copies the new scales into them at the loop's
// back edge, a copy that waits for every load in flight -- vmcnt(0) -- once per two groups, here and
// in t2_step. Passing the scales through the LDS tile instead, and giving each loop a single exit,
// removed every such wait and left the Qwen3-4B projections at 4, 16 and 24 tokens unchanged in
// total (-0.9% to +0.4%; +3 to +9% for gate/up, -2 to -9% for the others): the waits are not what
// bounds these kernels.)
template <int FMT, int TT>
__device__ __forceinline__ void mm_step(float4v (&acc)[TT], MmStage<FMT>& st, const half8 (&A)[kGroup][TT],
                                        half8 (&A_next)[kGroup][TT], const uint8_t* const (&prow)[pieces(FMT)],
                                        int col16, const uint8_t* wrow, int soff, const half_t* const (&xr)[TT], int g,
                                        int n, uint8_t* tile, const int (&slot)[pieces(FMT)], int b_acts, int b_stage) {
    load_acts<FMT, TT>(A_next, xr, b_acts, g);
    wave_sync_lds();  // the previous group's operand reads are done
#pragma unroll
    for (int q = 0; q < pieces(FMT); q++) *reinterpret_cast<uint4v*>(tile + slot[q]) = st.w[q];
    const uint2v sc = st.s;
    load_stage<FMT>(st, prow, col16, wrow, soff, b_stage);
    wave_sync_lds();
#pragma unroll
    for (int j = 0; j < kGroup; j++) {
        float s = 0.0f;
        if constexpr (FMT != 0) {
            // Copied out first: hipcc miscompiles __builtin_bit_cast of a vector element expression
            // (it reads element 0 whatever the index).
            const uint32_t sw = sc[j >> 1];
            const half2v s2 = __builtin_bit_cast(half2v, sw);
            s = static_cast<float>(s2[j & 1]) * block_scale_factor<FMT>();
        }
        mma_block<FMT, TT>(acc, A[j], decode_b<FMT>(read_b<FMT>(tile, n, j, g)), s);
    }
}

// Waves per workgroup the kernel is compiled for: more than one token tile needs more than 128
// VGPRs, which allows at most 8 waves.
__host__ __device__ constexpr int max_waves(int /*fmt*/, int tt) { return tt == 1 ? 16 : 8; }

// Dynamic LDS of a workgroup: the waves' staging tiles and, with more than one wave, the partial
// tiles of the K split.
__host__ __device__ constexpr size_t tile_lds_bytes(int fmt, int waves, int tt) {
    return static_cast<size_t>(waves) * stage_bytes(fmt) + (waves > 1 ? static_cast<size_t>(waves) * tt * 64 * 16 : 0);
}

// Grid: x = tiles of 16 weight rows, y = chunks of 16*TT tokens. Block: 64 * waves threads; wave w
// takes K blocks [w * blocks_per_wave, ...). Dynamic LDS: one staging tile per wave, then
// waves * TT * 64 float4 partial tiles.
template <int FMT, int TT, typename TY>
__global__ __launch_bounds__(64 * max_waves(FMT, TT)) void mm_tile_kernel(MmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int G = kGroup, NP = pieces(FMT), PR = group_row_bytes(FMT) / 16;  // pieces per row
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // uniform: scalar loop control
    const int waves = static_cast<int>(blockDim.x) >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int64_t t_base = static_cast<int64_t>(blockIdx.y) * (16 * TT);
    const int64_t last = a.N - 1;
    const uint8_t* wrow = a.w + min(row0 + n, last) * a.rb;
    const int soff = FMT == 1 ? a.K : a.K / 2;  // scale area of FP8 / FP4 rows
    uint8_t* tile = lds + wave * stage_bytes(FMT);

    // This lane's staging pieces: rows and LDS slots (fixed for every group).
    const uint8_t* prow[NP];
    int slot[NP];
    const int col16 = lane % PR;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = (64 * i + lane) / PR;
        prow[i] = a.w + min(row0 + r, last) * a.rb;
        slot[i] = r * stage_row(FMT) + col16 * 16;
    }

    const half_t* xr[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int64_t t = t_base + tt * 16 + n;
        xr[tt] = static_cast<const half_t*>(a.x) + (t < a.T ? t : 0) * a.xs;
    }

    const int nblk = a.K / kBlockK;
    const int b_begin = wave * a.blocks_per_wave;
    const int b_end = min(nblk, b_begin + a.blocks_per_wave);
    float4v acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) acc[tt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    const int nfull = (b_end - b_begin) / G;  // whole groups of this wave's K slice
    if (nfull > 0) {
        // Two register sets (weights + activations) alternate, so no register with a load in
        // flight is ever copied. Issue order per step: the next group's activations, this group's
        // LDS write, the weights two groups ahead, this group's MFMAs -- every wait covers only the
        // group being computed. Requests past the last group re-read it (from L2): the number of
        // loads in flight is the same on every path, so the compiler's waits stay partial.
        const int lastg = nfull - 1;
        MmStage<FMT> st0, st1;
        half8 A0[G][TT], A1[G][TT];
        load_stage<FMT>(st0, prow, col16, wrow, soff, b_begin);
        load_stage<FMT>(st1, prow, col16, wrow, soff, b_begin + min(1, lastg) * G);
        load_acts<FMT, TT>(A0, xr, b_begin, g);
        for (int i = 0;; i += 2) {
            mm_step<FMT, TT>(acc, st0, A0, A1, prow, col16, wrow, soff, xr, g, n, tile, slot,
                             b_begin + min(i + 1, lastg) * G, b_begin + min(i + 2, lastg) * G);
            if (i + 1 >= nfull) break;
            mm_step<FMT, TT>(acc, st1, A1, A0, prow, col16, wrow, soff, xr, g, n, tile, slot,
                             b_begin + min(i + 2, lastg) * G, b_begin + min(i + 3, lastg) * G);
            if (i + 2 >= nfull) break;
        }
    }
    for (int b = b_begin + nfull * G; b < b_end; b++) {  // K tail of fewer than a group: direct loads
        half8 A[TT];
        const half8 B = decode_b<FMT>(load_b_raw<FMT>(wrow, b, g));
#pragma unroll
        for (int tt = 0; tt < TT; tt++) A[tt] = load_a<FMT>(xr[tt], b, g);
        float s = 0.0f;
        if constexpr (FMT != 0)
            s = static_cast<float>(*reinterpret_cast<const half_t*>(wrow + soff + 2 * b)) * block_scale_factor<FMT>();
        mma_block<FMT, TT>(acc, A, B, s);
    }

    if (waves > 1) {
        float4v* red = reinterpret_cast<float4v*>(lds + waves * stage_bytes(FMT));
#pragma unroll
        for (int tt = 0; tt < TT; tt++) red[(wave * TT + tt) * 64 + lane] = acc[tt];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            float4v s = red[tt * 64 + lane];
            for (int w = 1; w < waves; w++) s += red[(w * TT + tt) * 64 + lane];
            acc[tt] = s;
        }
    }
    // Lane (n, g) holds C[token 4g + i][row n] of each 16 x 16 tile.
    const int64_t out_row = row0 + n;
    if (out_row >= a.N) return;
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t t = t_base + tt * 16 + 4 * g + i;
            if (t < a.T) epilogue<TY>(a, t, out_row, acc[tt][i]);
        }
    }
}

// ---------------------------------------------------------------- prefill GEMM, F16, direct-to-LDS loads
//
// F16 rows on large grids: 256 x 256 workgroup tiles over eight waves of 128 x 64 (4 x 2
// v_mfma_f32_32x32x16_f16 tiles, 128 accumulators per lane) at two waves per SIMD, K staged 64 at a
// time in double-buffered LDS (128 KB). Operands go from global memory straight into LDS
// (global_load_lds_dwordx4: lane l of an instruction writes bytes [16 l, 16 l + 16) past the wave's
// LDS base), so no staging registers are needed -- with them the 128 accumulators spill. Each
// instruction fills 8 unpadded 128-byte rows; within a row, 16-byte chunk c sits at slot
// c ^ ((row / 2) % 8), so the 16 rows one ds_read_b128 pass serves fall on distinct bank groups.
// A stage's loads are issued before the previous stage's MFMAs and waited for (vmcnt) before the
// barrier that publishes them.
constexpr int kG3GroupM = 8;  // token tiles per group of the XCD-contiguous tile walk
constexpr int kG3BM = 256, kG3BN = 256, kG3Threads = 512;

struct Gemm3Lds {
    half_t a[2][kG3BM * 64];
    half_t b[2][kG3BN * 64];
};

__device__ __forceinline__ int g3_slot(int row, int c) { return c ^ ((row >> 1) & 7); }

static_assert(sizeof(Gemm3Lds) >= (kG3Threads / 64) * kTileLdsFloats * sizeof(float), "epilogue scratch");

template <typename TY>
__global__ __launch_bounds__(kG3Threads, 2) void mm_gemm3_kernel(MmArgs a, int tiles_m, int tiles_n) {
    extern __shared__ __align__(16) uint8_t g3_lds[];
    Gemm3Lds& L = *reinterpret_cast<Gemm3Lds*>(g3_lds);
    constexpr int TM = 4, TN = 2;
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 1, wn = wave >> 1;

    uint32_t b = blockIdx.x;
    const uint32_t nb = gridDim.x;
    if (nb % 8 == 0) b = (b % 8) * (nb / 8) + b / 8;
    constexpr int GM = kG3GroupM;
    const int group = static_cast<int>(b) / (GM * tiles_n);
    const int first_m = group * GM, gm = min(GM, tiles_m - first_m);
    const int in_group = static_cast<int>(b) - group * GM * tiles_n;
    const int64_t m0 = static_cast<int64_t>(first_m + in_group % gm) * kG3BM;
    const int64_t n0 = static_cast<int64_t>(in_group / gm) * kG3BN;

    // This lane's four load instructions per operand and stage: rows (4 wave + i) * 8 + lane / 8, the
    // global chunk whose swizzled slot is lane % 8.
    const half_t* xa[4];
    const uint8_t* wb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (wave * 4 + i) * 8 + (lane >> 3), c = g3_slot(row, lane & 7);
        xa[i] = static_cast<const half_t*>(a.x) + min(m0 + row, a.T - 1) * a.xs + 8 * c;
        wb[i] = a.w + min(n0 + row, static_cast<int64_t>(a.N) - 1) * a.rb + 16 * c;
    }
    auto issue = [&](int k0, int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r0 = (wave * 4 + i) * 8;
            // (address-space conversions: C casts, which reinterpret_cast does not allow)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(xa[i] + k0),
                                             (__attribute__((address_space(3))) void*)(&L.a[buf][r0 * 64]), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(wb[i] + 2 * k0),
                                             (__attribute__((address_space(3))) void*)(&L.b[buf][r0 * 64]), 16, 0, 0);
        }
    };

    float16v acc[TM][TN] = {};
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = a.K / 64;
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int buf = s & 1;
        if (s + 1 < nk) issue((s + 1) * 64, buf ^ 1);  // that buffer's last readers passed the barrier
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            half8 B[TN][2];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int r = wn * 64 + j * 32 + l32;
#pragma unroll
                for (int q = 0; q < 2; q++)
                    B[j][q] = *reinterpret_cast<const half8*>(&L.b[buf][r * 64 + 8 * g3_slot(r, 4 * bb + 2 * q + h)]);
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int r = wm * 128 + i * 32 + l32;
                half8 A[2];
#pragma unroll
                for (int q = 0; q < 2; q++)
                    A[q] = *reinterpret_cast<const half8*>(&L.a[buf][r * 64 + 8 * g3_slot(r, 4 * bb + 2 * q + h)]);
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], acc[i][j], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the next stage have landed
        __syncthreads();                // and every wave's; this stage's reads are done
    }
    // The operand buffers are free once every wave is past its last stage: each wave regroups its
    // tiles through its own slice of them.
    __syncthreads();
    store_tiles<TY, TM, TN>(a, acc, reinterpret_cast<float*>(g3_lds) + wave * kTileLdsFloats, m0 + wm * 128, n0 + wn * 64, lane);
}

template <typename TY>
int launch_gemm3(neko_hip_ctx* ctx, dim3 grid, const MmArgs& a, int tm, int tn) {
    constexpr size_t lds = sizeof(Gemm3Lds);
    static std::atomic<uint64_t> allowed{0};
    if (int rc = allow_lds(ctx, reinterpret_cast<const void*>(&mm_gemm3_kernel<TY>), lds, allowed)) return rc;
    hipLaunchKernelGGL((mm_gemm3_kernel<TY>), grid, dim3(kG3Threads), lds, ctx->stream, a, tm, tn);
    return NEKO_OK;
}

// ---------------------------------------------------------------- prefill GEMM, FP8 / FP4, direct-to-LDS loads
//
// The F16 kernel's tiling and pipeline (256 x 256 tiles, eight waves of 128 x 64, K staged 64 at a time
// in double-buffered LDS filled by global_load_lds) for code rows: the activations land in LDS exactly
// as there; the stage's raw codes land chunk-major -- 16-byte chunk c of row r at (c * 256 + r) * 16, so
// the 32 rows a read serves are contiguous and conflict-free -- and each row's two f16 block scales as
// one dword. Every wave decodes its own B fragments from the codes (FP8 by the bit trick, FP4 by
// v_cvt_scalef32_pk_f16_fp4; exact f16 values), sums each 32-wide block with two MFMAs from zero and
// adds it into the accumulators scaled by the block's f32 scale (one fma per output per block), as the
// register-staged kernel does.

template <int FMT>
struct Gemm3qLds {
    static constexpr int KC = FMT == 1 ? 4 : 2;  // 16-byte code chunks per row and stage
    half_t a[2][kG3BM * 64];
    uint8_t b[2][KC * kG3BN * 16];
    uint32_t s[2][kG3BN];
};

// FP4 byte SEL of word q -> its two weights as f16 (low nibble first); SEL must be a literal.
#define NEKO_FP4_PAIR3(q, SEL) __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4((q), 1.0f, SEL))

// The two B operands (k 0..15 and 16..31 of block bb, this lane's 8 of each) of row r.
template <int FMT>
__device__ __forceinline__ void g3q_read_b(const uint8_t* lb, int bb, int r, int h, half8 (&B)[2]) {
    if constexpr (FMT == 1) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const uint2v w = *reinterpret_cast<const uint2v*>(lb + ((2 * bb + q) * kG3BN + r) * 16 + 8 * h);
            uint4v o;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                o[2 * i] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w[i], 0x0C010C00u));
                o[2 * i + 1] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w[i], 0x0C030C02u));
            }
            B[q] = __builtin_bit_cast(half8, o);
        }
    } else {
        // Bytes 8 h .. 8 h + 7 of the block: weights 8 h + j (low nibbles) and 16 + 8 h + j (high).
        const uint2v w = *reinterpret_cast<const uint2v*>(lb + (bb * kG3BN + r) * 16 + 8 * h);
        uint32_t pr[8];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            pr[4 * i] = NEKO_FP4_PAIR3(w[i], 0);
            pr[4 * i + 1] = NEKO_FP4_PAIR3(w[i], 1);
            pr[4 * i + 2] = NEKO_FP4_PAIR3(w[i], 2);
            pr[4 * i + 3] = NEKO_FP4_PAIR3(w[i], 3);
        }
        uint4v lo, hi;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            lo[j] = __builtin_amdgcn_perm(pr[2 * j + 1], pr[2 * j], 0x05040100u);
            hi[j] = __builtin_amdgcn_perm(pr[2 * j + 1], pr[2 * j], 0x07060302u);
        }
        B[0] = __builtin_bit_cast(half8, lo);
        B[1] = __builtin_bit_cast(half8, hi);
    }
}
#undef NEKO_FP4_PAIR3

template <int FMT, typename TY>
__global__ __launch_bounds__(kG3Threads, 2) void mm_gemm3q_kernel(MmArgs a, int tiles_m, int tiles_n) {
    typedef Gemm3qLds<FMT> Lds;
    constexpr int KC = Lds::KC, NB = KC / 2;  // B load instructions per lane and stage
    static_assert(sizeof(Lds) >= (kG3Threads / 64) * kTileLdsFloats * sizeof(float), "epilogue scratch");
    extern __shared__ __align__(16) uint8_t g3_lds[];
    Lds& L = *reinterpret_cast<Lds*>(g3_lds);
    constexpr int TM = 4, TN = 2;
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 1, wn = wave >> 1;

    uint32_t b = blockIdx.x;
    const uint32_t nb = gridDim.x;
    if (nb % 8 == 0) b = (b % 8) * (nb / 8) + b / 8;
    constexpr int GM = kG3GroupM;
    const int group = static_cast<int>(b) / (GM * tiles_n);
    const int first_m = group * GM, gm = min(GM, tiles_m - first_m);
    const int in_group = static_cast<int>(b) - group * GM * tiles_n;
    const int64_t m0 = static_cast<int64_t>(first_m + in_group % gm) * kG3BM;
    const int64_t n0 = static_cast<int64_t>(in_group / gm) * kG3BN;
    const int64_t lastN = static_cast<int64_t>(a.N) - 1;

    // Activations: as mm_gemm3_kernel (rows (4 wave + i) * 8 + lane / 8, swizzled chunk slots).
    const half_t* xa[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (wave * 4 + i) * 8 + (lane >> 3), c = g3_slot(row, lane & 7);
        xa[i] = static_cast<const half_t*>(a.x) + min(m0 + row, a.T - 1) * a.xs + 8 * c;
    }
    // Codes: this lane's chunk p = (wave NB + i) 64 + lane of the stage, chunk p / 256 of row p % 256.
    const uint8_t* wb[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int p = (wave * NB + i) * 64 + lane, c = p / kG3BN, r = p % kG3BN;
        wb[i] = a.w + min(n0 + r, lastN) * a.rb + 16 * c;
    }
    // Scales: waves 0-3, lane l: row 64 wave + l.
    const uint8_t* ws = a.w + min(n0 + 64 * (wave & 3) + lane, lastN) * a.rb + (FMT == 1 ? a.K : a.K / 2);
    auto issue = [&](int k0, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r0 = (wave * 4 + i) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(xa[i] + k0),
                                             (__attribute__((address_space(3))) void*)(&L.a[buf][r0 * 64]), 16, 0, 0);
        }
        const int kb = FMT == 1 ? k0 : k0 / 2;  // code bytes before the stage
#pragma unroll
        for (int i = 0; i < NB; i++)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(wb[i] + kb),
                                             (__attribute__((address_space(3))) void*)(&L.b[buf][(wave * NB + i) * 64 * 16]), 16, 0, 0);
        if (wave < 4)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(ws + 2 * (k0 / kBlockK)),
                                             (__attribute__((address_space(3))) void*)(&L.s[buf][64 * wave]), 4, 0, 0);
    };

    float16v acc[TM][TN] = {};
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = a.K / 64;
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int buf = s & 1;
        if (s + 1 < nk) issue((s + 1) * 64, buf ^ 1);  // that buffer's last readers passed the barrier
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            half8 B[TN][2];
            float sc[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int r = wn * 64 + j * 32 + l32;
                g3q_read_b<FMT>(L.b[buf], bb, r, h, B[j]);
                const half2v s2 = __builtin_bit_cast(half2v, L.s[buf][r]);
                // FP8 codes decode to value / 2^8; FP4 through the hardware conversion (exact values).
                sc[j] = static_cast<float>(s2[bb]) * block_scale_factor<FMT>();
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int r = wm * 128 + i * 32 + l32;
                half8 A[2];
#pragma unroll
                for (int q = 0; q < 2; q++)
                    A[q] = *reinterpret_cast<const half8*>(&L.a[buf][r * 64 + 8 * g3_slot(r, 4 * bb + 2 * q + h)]);
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    float16v blk = {};
                    blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], blk, 0, 0, 0);
                    blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], blk, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][j][e] = __builtin_fmaf(sc[j], blk[e], acc[i][j][e]);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the next stage have landed
        __syncthreads();                // and every wave's; this stage's reads are done
    }
    // The operand buffers are free once every wave is past its last stage: each wave regroups its
    // tiles through its own slice of them.
    __syncthreads();
    store_tiles<TY, TM, TN>(a, acc, reinterpret_cast<float*>(g3_lds) + wave * kTileLdsFloats, m0 + wm * 128, n0 + wn * 64, lane);
}

template <int FMT, typename TY>
int launch_gemm3q(neko_hip_ctx* ctx, dim3 grid, const MmArgs& a, int tm, int tn) {
    constexpr size_t lds = sizeof(Gemm3qLds<FMT>);
    static std::atomic<uint64_t> allowed{0};
    if (int rc = allow_lds(ctx, reinterpret_cast<const void*>(&mm_gemm3q_kernel<FMT, TY>), lds, allowed)) return rc;
    hipLaunchKernelGGL((mm_gemm3q_kernel<FMT, TY>), grid, dim3(kG3Threads), lds, ctx->stream, a, tm, tn);
    return NEKO_OK;
}

// ---------------------------------------------------------------- mid-size T: activations shared in LDS
//
// FP4 at 5 <= T < 48, FP8 at 13 <= T < 48, F16 at 17 <= T < 33: second form: each wave of a 4-wave workgroup
// owns its own 16-row tile, and the workgroup stages its token chunk's activations for one slice of
// K in LDS once, with coalesced loads (FP4 blocks pre-permuted to the MFMA k order), so every wave
// reads its A fragments from LDS. (Re-reading them from L1 per wave and group, 16 token rows per instruction, left the L1 tag
// lookups at their issue rate -- measured.) Weights stream through each wave's LDS staging tile as
// in mm_tile_kernel. K is split over the grid's z: with several slices the waves write f32 partials
// that mm_splitk_reduce adds in order. (Adding them in the kernel, by the last workgroup of each row
// group to arrive, measured several times slower: the device-scope fences that publish the partials
// write back / invalidate an XCD's whole L2. Without fences -- partials stored and re-read as
// device-scope relaxed atomics, which go past the XCD's L2, and a device-scope arrival counter --
// it was still slower on every Qwen3-4B projection at 16 and 24 tokens: FP8 down 16.7 -> 22.0 us,
// FP4 o 11.1 -> 14.0, against the launch it saves.)
constexpr int kT2Waves = 4;
constexpr int kT2Lds = 65536;  // LDS per workgroup (two per CU at 64 KB)
constexpr int64_t kT2MaxT = 48;  // exclusive; at most 65 (four 16-token tiles)
static_assert(kT2MaxT <= 65, "the shared-activation kernel holds at most 64 tokens");
constexpr int kT2Fill = 4;  // K slices until the grid holds this many workgroups per CU
// Token counts above which each format takes this kernel (below: the per-wave tile kernel).
constexpr int64_t kT2MinF16 = 16, kT2MinFp8 = 12, kT2MinFp4 = 4;


// Halves per staged token row for nb blocks: 32 nb plus 8 of padding (16-byte bank groups differ
// between the 16 token rows a ds_read_b128 pass serves: the row stride over 16 is odd).
__host__ __device__ constexpr int t2_row(int nb) { return 32 * nb + 8; }

// Bytes of the staged activations: `rows` token rows (the chunk's tokens, at most 16 TT) of nb blocks.
__host__ __device__ constexpr size_t t2_acts_bytes(int rows, int nb) { return static_cast<size_t>(rows) * t2_row(nb) * 2; }

// xoff[tt]: halves from the staged activations to this lane's token row of tile tt. Token rows past
// the chunk's last token read that token's row (a broadcast, no extra bank traffic); their MFMA
// output rows are never stored.
template <int FMT, int TT>
__device__ __forceinline__ void t2_load_acts(half8 (&A)[kGroup][TT], const half_t* xl, const int (&xoff)[TT], int b0, int g) {
#pragma unroll
    for (int j = 0; j < kGroup; j++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
            A[j][tt] = *reinterpret_cast<const half8*>(xl + xoff[tt] + (b0 + j) * kBlockK + 8 * g);
}

// One group, as mm_step, with the next group's activation fragments read from LDS.
template <int FMT, int TT>
__device__ __forceinline__ void t2_step(float4v (&acc)[TT], MmStage<FMT>& st, const half8 (&A)[kGroup][TT],
                                        half8 (&A_next)[kGroup][TT], const uint8_t* const (&prow)[pieces(FMT)],
                                        int col16, const uint8_t* wrow, int soff, const half_t* xl, const int (&xoff)[TT],
                                        int g, int n, uint8_t* tile, const int (&slot)[pieces(FMT)], int b_acts_rel,
                                        int b_stage) {
    t2_load_acts<FMT, TT>(A_next, xl, xoff, b_acts_rel, g);
    wave_sync_lds();  // the previous group's operand reads are done
#pragma unroll
    for (int q = 0; q < pieces(FMT); q++) *reinterpret_cast<uint4v*>(tile + slot[q]) = st.w[q];
    const uint2v sc = st.s;
    load_stage<FMT>(st, prow, col16, wrow, soff, b_stage);
    wave_sync_lds();
#pragma unroll
    for (int j = 0; j < kGroup; j++) {
        float s = 0.0f;
        if constexpr (FMT != 0) {
            const uint32_t sw = sc[j >> 1];  // copied out first (see mm_step)
            const half2v s2 = __builtin_bit_cast(half2v, sw);
            s = static_cast<float>(s2[j & 1]) * block_scale_factor<FMT>();
        }
        mma_block<FMT, TT>(acc, A[j], decode_b<FMT>(read_b<FMT>(tile, n, j, g)), s);
    }
}

// Grid: x = groups of 4 row tiles (64 rows), y = chunks of 16 TT tokens, z = K slices of
// `slice_blocks` blocks. Dynamic LDS: the staged activations (one row of t2_row(slice_blocks) halves
// per token of the chunk, at most 16 TT), then one weight staging tile per wave.
template <int FMT, int TT, typename TY>
__global__ __launch_bounds__(64 * kT2Waves) void mm_tile2_kernel(MmArgs a, int slice_blocks, float* partial,
                                                                  FastDiv div_full, FastDiv div_last) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int G = kGroup, NP = pieces(FMT), PR = group_row_bytes(FMT) / 16;
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kT2Waves + wave) * 16;
    const int64_t t_base = static_cast<int64_t>(blockIdx.y) * (16 * TT);
    const int nblk = a.K / kBlockK;
    const int kb0 = static_cast<int>(blockIdx.z) * slice_blocks;
    const int nb = min(nblk - kb0, slice_blocks);  // > 0: the host sizes the slices
    const int xr_stride = t2_row(slice_blocks);
    const int rows = static_cast<int>(min<int64_t>(16 * TT, a.T - t_base));  // tokens of this chunk
    half_t* xl = reinterpret_cast<half_t*>(lds);
    uint8_t* tile = lds + t2_acts_bytes(rows, slice_blocks) + wave * stage_bytes(FMT);
    int xoff[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) xoff[tt] = min(tt * 16 + n, rows - 1) * xr_stride;

    const int64_t last = a.N - 1;
    const uint8_t* wrow = a.w + min(row0 + n, last) * a.rb;
    const int soff = FMT == 1 ? a.K : a.K / 2;
    const uint8_t* prow[NP];
    int slot[NP];
    const int col16 = lane % PR;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = (64 * i + lane) / PR;
        prow[i] = a.w + min(row0 + r, last) * a.rb;
        slot[i] = r * stage_row(FMT) + col16 * 16;
    }
    // The first two groups' weights do not depend on the activations: requested before staging them.
    const int nfull = nb / G, lastg = max(nfull - 1, 0);
    MmStage<FMT> st0, st1;
    if (nfull > 0) {
        load_stage<FMT>(st0, prow, col16, wrow, soff, kb0);
        load_stage<FMT>(st1, prow, col16, wrow, soff, kb0 + min(1, lastg) * G);
    }

    // Stage the activations: 16-byte chunk c = (token, block, h) holds halves 8h .. 8h+7 of the block.
    // FP4 groups lane g's k set {4g..4g+3, 16+4g..16+4g+3} at halves 8g .. 8g+7 of the staged block.
    // Eight chunks per thread are requested before any is stored (one memory round trip per batch;
    // chunk indices past the end re-read the last chunk and are not stored).
    constexpr int kBatch = 8, kThreads = 64 * kT2Waves;
    const int chunks = rows * nb * 4;
    const FastDiv per_row = nb == slice_blocks ? div_full : div_last;  // chunk -> token: by nb * 4
    for (int c0 = tid; c0 < chunks; c0 += kThreads * kBatch) {
        uint4v v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
            const int c = min(c0 + kThreads * u, chunks - 1);
            const int t = static_cast<int>(fast_div(static_cast<uint32_t>(c), per_row)), q = c - t * (nb * 4);
            const int64_t tok = t_base + t;  // t < rows
            v[u] = *reinterpret_cast<const uint4v*>(static_cast<const half_t*>(a.x) + tok * a.xs + kb0 * kBlockK + 8 * q);
        }
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
            const int c = c0 + kThreads * u;
            if (c >= chunks) break;
            const int t = static_cast<int>(fast_div(static_cast<uint32_t>(c), per_row));
            const int q = c - t * (nb * 4), b = q >> 2, h = q & 3;
            half_t* dst = xl + t * xr_stride + b * kBlockK;
            if constexpr (FMT == 2) {
                // Chunk h covers k 8h .. 8h+7: its halves k 8h..8h+3 and 8h+4..8h+7 belong to groups
                // 2 (h & 1) and 2 (h & 1) + 1, in their low (h < 2) or high (h >= 2) four halves.
                const int g0 = 2 * (h & 1), hi = 4 * (h >> 1);
                *reinterpret_cast<uint2v*>(dst + 8 * g0 + hi) = uint2v{v[u][0], v[u][1]};
                *reinterpret_cast<uint2v*>(dst + 8 * (g0 + 1) + hi) = uint2v{v[u][2], v[u][3]};
            } else {
                *reinterpret_cast<uint4v*>(dst + 8 * h) = v[u];
            }
        }
    }
    __syncthreads();

    float4v acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) acc[tt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    if (nfull > 0) {
        half8 A0[G][TT], A1[G][TT];
        t2_load_acts<FMT, TT>(A0, xl, xoff, 0, g);
        for (int i = 0;; i += 2) {
            t2_step<FMT, TT>(acc, st0, A0, A1, prow, col16, wrow, soff, xl, xoff, g, n, tile, slot,
                             min(i + 1, lastg) * G, kb0 + min(i + 2, lastg) * G);
            if (i + 1 >= nfull) break;
            t2_step<FMT, TT>(acc, st1, A1, A0, prow, col16, wrow, soff, xl, xoff, g, n, tile, slot,
                             min(i + 2, lastg) * G, kb0 + min(i + 3, lastg) * G);
            if (i + 2 >= nfull) break;
        }
    }
    for (int b = nfull * G; b < nb; b++) {  // K tail of fewer than a group: direct weight loads
        half8 A[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
            A[tt] = *reinterpret_cast<const half8*>(xl + xoff[tt] + b * kBlockK + 8 * g);
        const half8 B = decode_b<FMT>(load_b_raw<FMT>(wrow, kb0 + b, g));
        float s = 0.0f;
        if constexpr (FMT != 0)
            s = static_cast<float>(*reinterpret_cast<const half_t*>(wrow + soff + 2 * (kb0 + b))) * block_scale_factor<FMT>();
        mma_block<FMT, TT>(acc, A, B, s);
    }

    // Lane (n, g) holds C[token 4g + i][row n] of each 16 x 16 tile.
    const int64_t out_row = row0 + n;
    if (out_row >= a.N) return;
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t t = t_base + tt * 16 + 4 * g + i;
            if (t >= a.T) continue;
            if (partial) partial[(static_cast<int64_t>(blockIdx.z) * a.T + t) * a.N + out_row] = acc[tt][i];
            else epilogue<TY>(a, t, out_row, acc[tt][i]);
        }
}

// ---------------------------------------------------------------- decode path: VALU GEMV

// Sum over each DPP row of 16 lanes; every lane of the row receives the same bits.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    return v;
}

// Staged activation rows: 16 bytes of padding after every 256 bytes of blocks (every 4 f16 / 2 f32
// blocks). The 16 lanes of a weight row read the same 16-byte chunk of 16 consecutive blocks in one
// instruction: unpadded, those addresses are 64 / 128 bytes apart and fall on 4 / 2 of LDS's sixteen
// 16-byte bank groups (4- / 8-way conflicts); padded they take all sixteen, for any first block,
// and every chunk read keeps a constant offset from its block's address. Measured at 1-4 tokens on
// the Qwen3-4B projections against unpadded rows: f32 activations 1.2-2.5x faster (FP4 gate/up
// 19.3 -> 12.2 us at one token, 54.6 -> 22.2 at four), f16 up to 11% (FP4 gate/up at two tokens
// 14.4 -> 12.8 us; FP8 within 0.3 us either way). An XOR swizzle of the chunks instead (no padding)
// gained less for f32 and cost time for f16: its per-read address arithmetic.
__host__ __device__ constexpr int gemv_blk_off(int blk, int x_bytes) {  // element offset of block blk
    return blk * 32 + (blk >> (x_bytes == 4 ? 1 : 2)) * (16 / x_bytes);
}

// Two weights as f16 (exact values / 2^8 for FP8, the values for FP4) paired with the activation
// pair at the same positions of the staged x block; dot of one 32-wide block against token t. f16
// activations: one fdot2 per pair; f32 activations (the reference's own type): one fma per weight,
// the f16 weight widened exactly.
template <int FMT, typename TX>
__device__ __forceinline__ float block_dot(const uint4v (&q)[FMT == 0 ? 4 : FMT == 1 ? 2 : 1], const TX* xb) {
    float d = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {  // 4 x 8 activations
        uint32_t wp[4];
        if constexpr (FMT == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) wp[i] = q[c][i];
        } else if constexpr (FMT == 1) {
            const uint32_t w0 = q[c >> 1][(c & 1) * 2], w1 = q[c >> 1][(c & 1) * 2 + 1];
            wp[0] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w0, 0x0C010C00u));
            wp[1] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w0, 0x0C030C02u));
            wp[2] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w1, 0x0C010C00u));
            wp[3] = fp8_pair_bits(__builtin_amdgcn_perm(0u, w1, 0x0C030C02u));
        } else {
            // Bytes 4c .. 4c+3 of the block: (weight j, weight 16 + j) pairs, matching the staged
            // x order (x_j, x_16+j).
            const uint32_t w = q[0][c];
            wp[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0));
            wp[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1));
            wp[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2));
            wp[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3));
        }
        if constexpr (sizeof(TX) == 2) {
            const uint4v xc = reinterpret_cast<const uint4v*>(xb)[c];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t xw = xc[i];
                d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, wp[i]), __builtin_bit_cast(half2v, xw), d, false);
            }
        } else {
            const float4v x0 = reinterpret_cast<const float4v*>(xb)[2 * c], x1 = reinterpret_cast<const float4v*>(xb)[2 * c + 1];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const half2v w2 = __builtin_bit_cast(half2v, wp[i]);
                const float xa = i < 2 ? x0[2 * i] : x1[2 * i - 4], xb2 = i < 2 ? x0[2 * i + 1] : x1[2 * i - 3];
                d = __builtin_fmaf(xa, static_cast<float>(w2[0]), d);
                d = __builtin_fmaf(xb2, static_cast<float>(w2[1]), d);
            }
        }
    }
    return d;
}

// Largest T taking the GEMV path: 2 (measured on the Qwen3-4B projections: at 3 and 4 tokens the
// MFMA tile kernels take 14% less time over the four projections, at 2 the GEMV 11% less).
constexpr int64_t kGemvMaxT = 2;
static_assert(kGemvMaxT >= 1 && kGemvMaxT <= 4, "the GEMV holds 1, 2 or 4 tokens per pass");
constexpr int64_t kGemvWaveTarget = 8192;
// f32 activations (the reference's own type, as its ComputeBackend passes them) take the GEMV below
// the two-plane split's threshold, and at any T its grid holds where the split cannot run (the
// allocation-free entry): the MFMA kernels read f16 activations, and the GEMV's NT-token passes beat
// the generic kernel's per-element loads at every T measured (4.9-7.4x at one token).
constexpr int64_t kGemv32MaxT = 65535;
constexpr int kGemvRows = 4;    // weight rows per wave: 16 lanes each
constexpr int kGemvWaves = 8;   // waves per workgroup: (8 / kw) row groups x kw slices of K
constexpr int kGemvBatch = 2;  // 32-wide blocks per lane whose weights are requested together

// Grid: x = workgroups of 4 * 8 / kw weight rows, y = chunks of NT tokens. Wave w works on row
// group w / kw and K slice w % kw (a.blocks_per_wave blocks). Dynamic LDS: the chunk's activations as TX [NT][xrow], rows padded as above (FP4: each 32-block
// stored as (x_j, x_16+j) pairs), then 8 * 4 * NT partial sums.
template <int FMT, int NT, typename TY, typename TX>
__global__ __launch_bounds__(64 * kGemvWaves) void mm_gemv_kernel(MmArgs a, int kw) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NW = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;  // 16-byte weight loads per block
    constexpr int U = kGemvBatch;
    constexpr int EPC = 16 / static_cast<int>(sizeof(TX));  // activations per 16-byte piece
    TX* xs = reinterpret_cast<TX*>(lds);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int rg = wave / kw, ks = wave - rg * kw;  // row group, K slice
    const int r = lane >> 4, sl = lane & 15;
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * NT;
    const int nt = static_cast<int>(min(static_cast<int64_t>(NT), a.T - t0));
    const int K = a.K;
    const int xrow = gemv_blk_off(K / kBlockK, sizeof(TX));  // staged row, elements

    const int64_t row = (static_cast<int64_t>(blockIdx.x) * (kGemvWaves / kw) + rg) * kGemvRows + r;
    const uint8_t* wrow = a.w + min(row, static_cast<int64_t>(a.N) - 1) * a.rb;
    const int soff = FMT == 1 ? K : K / 2;
    const int nblk = K / kBlockK;
    const int b_begin = min(nblk, ks * a.blocks_per_wave);
    const int b_end = min(nblk, b_begin + a.blocks_per_wave);
    const int steps = (b_end - b_begin + 15) / 16;  // wave-uniform; 0 for an empty slice
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;

    // Every wave runs at least one batch (the x staging and its barrier are in the first).
    for (int j0 = 0; j0 == 0 || j0 < steps; j0 += U) {
        uint4v q[U][NW];
        float sc[U];
        bool valid[U];
        int bl[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = b_begin + sl + 16 * (j0 + u);
            valid[u] = b < b_end;
            bl[u] = valid[u] ? b : max(b_begin, b_end - 1);  // in bounds and unconditional
            bl[u] = min(bl[u], nblk - 1);
#pragma unroll
            for (int i = 0; i < NW; i++)
                q[u][i] = *reinterpret_cast<const uint4v*>(wrow + bl[u] * block_bytes(FMT) + 16 * i);
            sc[u] = 1.0f;
            if constexpr (FMT != 0)
                sc[u] = static_cast<float>(*reinterpret_cast<const half_t*>(wrow + soff + 2 * bl[u])) *
                        block_scale_factor<FMT>();
        }
        if (j0 == 0) {
            // Stage x rows t0 .. t0 + NT - 1 (rows past T are zero) in 16-byte pieces, while the
            // first weights are in flight.
            const int kc = K / EPC;
            for (int i = static_cast<int>(threadIdx.x); i < NT * kc; i += static_cast<int>(blockDim.x)) {
                const int t = i / kc, c = i - t * kc;
                uint4v v = {0u, 0u, 0u, 0u};
                if (t < nt) v = *reinterpret_cast<const uint4v*>(static_cast<const TX*>(a.x) + (t0 + t) * a.xs + EPC * c);
                // Piece c: elements kb .. kb + EPC - 1 of block c * EPC / 32, at that block's padded offset.
                const int kb = (EPC * c) % kBlockK;
                TX* dst = xs + static_cast<int64_t>(t) * xrow + gemv_blk_off((EPC * c) / kBlockK, sizeof(TX));
                if constexpr (FMT == 2) {
                    // Element k of the block to 2 k (k < 16) or 2 (k - 16) + 1.
#pragma unroll
                    for (int e = 0; e < EPC; e++) {
                        const int k = kb + e;
                        TX val;
                        if constexpr (sizeof(TX) == 2) val = __builtin_bit_cast(half8, v)[e];
                        else val = __builtin_bit_cast(float4v, v)[e];
                        dst[k < 16 ? 2 * k : 2 * (k - 16) + 1] = val;
                    }
                } else {
                    *reinterpret_cast<uint4v*>(dst + kb) = v;
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (j0 + u >= steps) break;  // wave-uniform
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float d = block_dot<FMT, TX>(q[u], xs + static_cast<int64_t>(t) * xrow + gemv_blk_off(bl[u], sizeof(TX)));
                const float v = FMT == 0 ? d : d * sc[u];
                acc[t] += valid[u] ? v : 0.0f;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = row16_sum(acc[t]);

    if (kw > 1) {
        float* red = reinterpret_cast<float*>(lds + static_cast<size_t>(NT) * xrow * sizeof(TX));
        if (sl == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) red[(wave * kGemvRows + r) * NT + t] = acc[t];
        }
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float v = red[(wave * kGemvRows + r) * NT + t];
            for (int w = 1; w < kw; w++) v += red[((wave + w) * kGemvRows + r) * NT + t];
            acc[t] = v;
        }
    }
    if (row >= a.N || sl >= nt) return;
    float v = acc[0];
#pragma unroll
    for (int t = 1; t < NT; t++)
        if (sl == t) v = acc[t];
    epilogue<TY>(a, t0 + sl, row, v);
}

__host__ __device__ constexpr size_t gemv_lds_bytes(int K, int nt, int x_bytes = 2) {
    return static_cast<size_t>(nt) * gemv_blk_off(K / kBlockK, x_bytes) * x_bytes + static_cast<size_t>(kGemvWaves) * kGemvRows * nt * 4;
}

// ---------------------------------------------------------------- prefill path: MFMA GEMM

// Workgroup tile: BM tokens x BN weight rows (BM = 32 MF, BN = 32 NF), K in 32-wide steps (one
// FP8/FP4 scale block). Four waves in 2 x 2, each an (16 MF) x (16 NF) tile of
// v_mfma_f32_16x16x32_f16. Per step the workgroup stages the activation tile and the weight tile --
// codes decoded once to exact f16 values -- in double-buffered LDS; the next step's global loads are
// in flight during this step's MFMAs. LDS bytes per MFMA fall as the wave tile grows (both operand
// fragments are reused across the other dimension), which is what bounds a 64 x 64 wave tile.
// Smallest T taking the GEMM path: from 33 tokens for F16 rows, 48 for FP8 / FP4 (measured on the
// Qwen3-4B projections: below these the shared-activation kernel's three token tiles are faster).
constexpr int64_t kGemmMinT = 48;
constexpr int64_t kGemmMinTF16 = 33;
constexpr int kGemmMF = 4, kGemmNF = 4;  // 16-wide fragments per wave (two 32 x 32 MFMA tiles each way)
constexpr int kGemmWM = 2, kGemmWN = 2;  // waves per workgroup
constexpr int kGemmThreads = 64 * kGemmWM * kGemmWN;
constexpr int kGemmBM = 16 * kGemmMF * kGemmWM, kGemmBN = 16 * kGemmNF * kGemmWN, kGemmBK = 32;
constexpr int kGemmRow = 40;  // halves per LDS row: 32 plus 8 of padding (no bank conflicts)
static_assert(kGemmBN == kGemmThreads / 2, "the weight-tile load split: two threads per weight row");
static_assert((kGemmBM * 4) % kGemmThreads == 0, "activation pieces per thread");

// Half offset of 16-byte chunk c (0..3) of row r in a staged tile.
__device__ __forceinline__ int gemm_off(int r, int c) { return r * kGemmRow + 8 * c; }

struct GemmLds {
    half_t a[2][kGemmBM * kGemmRow];
    half_t b[2][kGemmBN * kGemmRow];
    float s[2][kGemmBN];  // the step's block scale of each row (times the decode factor)
};

template <int FMT>
struct GemmRegs {
    uint4v a[kGemmBM * 4 / kGemmThreads];                            // 16-byte activation pieces
    typename VecOf<uint32_t, FMT == 0 ? 8 : FMT == 1 ? 4 : 2>::V w;  // 32 / 16 / 8 weight bytes
    half_t s;
};

// Thread tid's pieces of step k0: activations rows (tid + 256 i) / 4, 16-byte column (tid % 4);
// weights: F16 the same split of 64-byte row blocks, FP8 row tid / 2 half tid % 2 (16 codes), FP4 row
// tid / 2 half tid % 2 (8 bytes); scales: thread tid < 128 takes row tid.
template <int FMT>
__device__ __forceinline__ void gemm_load(GemmRegs<FMT>& r, const MmArgs& a, int64_t m0, int64_t n0, int k0, int tid) {
    const int64_t lastT = a.T - 1, lastN = a.N - 1;
#pragma unroll
    for (int i = 0; i < kGemmBM * 4 / kGemmThreads; i++) {
        const int p = tid + kGemmThreads * i, row = p >> 2, c = p & 3;
        const half_t* xr = static_cast<const half_t*>(a.x) + min(m0 + row, lastT) * a.xs;
        r.a[i] = *reinterpret_cast<const uint4v*>(xr + k0 + 8 * c);
    }
    if constexpr (FMT == 0) {
        uint4v w[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int p = tid + kGemmThreads * i, row = p >> 2, c = p & 3;
            w[i] = *reinterpret_cast<const uint4v*>(a.w + min(n0 + row, lastN) * a.rb + 2 * (k0 + 8 * c));
        }
        r.w = __builtin_shufflevector(w[0], w[1], 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
        const int row = tid >> 1, h = tid & 1;
        const uint8_t* wr = a.w + min(n0 + row, lastN) * a.rb;
        const int bb = block_bytes(FMT);
        if constexpr (FMT == 1) r.w = *reinterpret_cast<const uint4v*>(wr + (k0 / kBlockK) * bb + 16 * h);
        else r.w = *reinterpret_cast<const uint2v*>(wr + (k0 / kBlockK) * bb + 8 * h);
        if (tid < kGemmBN) {
            const uint8_t* sr = a.w + min(n0 + tid, lastN) * a.rb + (FMT == 1 ? a.K : a.K / 2);
            r.s = *reinterpret_cast<const half_t*>(sr + 2 * (k0 / kBlockK));
        }
    }
}

template <int FMT>
__device__ __forceinline__ void gemm_store(GemmLds& L, int buf, const GemmRegs<FMT>& r, int tid) {
#pragma unroll
    for (int i = 0; i < kGemmBM * 4 / kGemmThreads; i++) {
        const int p = tid + kGemmThreads * i, row = p >> 2, c = p & 3;
        *reinterpret_cast<uint4v*>(&L.a[buf][gemm_off(row, c)]) = r.a[i];
    }
    if constexpr (FMT == 0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int p = tid + kGemmThreads * i, row = p >> 2, c = p & 3;
            const uint4v v = {r.w[4 * i], r.w[4 * i + 1], r.w[4 * i + 2], r.w[4 * i + 3]};
            *reinterpret_cast<uint4v*>(&L.b[buf][gemm_off(row, c)]) = v;
        }
    } else {
        const int row = tid >> 1, h = tid & 1;
        if constexpr (FMT == 1) {
            // 16 codes -> 16 halves at positions 16 h ..
            uint32_t o[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q = r.w[i];
                o[2 * i] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q, 0x0C010C00u));
                o[2 * i + 1] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q, 0x0C030C02u));
            }
            *reinterpret_cast<uint4v*>(&L.b[buf][gemm_off(row, 2 * h)]) = uint4v{o[0], o[1], o[2], o[3]};
            *reinterpret_cast<uint4v*>(&L.b[buf][gemm_off(row, 2 * h + 1)]) = uint4v{o[4], o[5], o[6], o[7]};
        } else {
            // Bytes 8 h .. 8 h + 7: byte i holds weights 8 h + i (low nibble) and 16 + 8 h + i (high):
            // the hardware conversion yields those pairs, regrouped into natural order.
            const uint32_t q0 = r.w[0], q1 = r.w[1];
            const uint32_t c[8] = {
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q0, 1.0f, 0)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q0, 1.0f, 1)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q0, 1.0f, 2)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q0, 1.0f, 3)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q1, 1.0f, 0)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q1, 1.0f, 1)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q1, 1.0f, 2)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(q1, 1.0f, 3))};
            uint4v lo, hi;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = __builtin_amdgcn_perm(c[2 * i + 1], c[2 * i], 0x05040100u);
                hi[i] = __builtin_amdgcn_perm(c[2 * i + 1], c[2 * i], 0x07060302u);
            }
            *reinterpret_cast<uint4v*>(&L.b[buf][gemm_off(row, h)]) = lo;
            *reinterpret_cast<uint4v*>(&L.b[buf][gemm_off(row, 2 + h)]) = hi;
        }
        if (tid < kGemmBN) L.s[buf][tid] = static_cast<float>(r.s) * block_scale_factor<FMT>();
    }
}

// The wave's (16 MF) x (16 NF) accumulator tile as 32 x 32 tiles (v_mfma_f32_32x32x16_f16: lane
// (l32, h) holds C[8 (v / 4) + 4 h + v % 4][l32] in register v). Measured on MI355X, independent
// 32 x 32 x 16 MFMAs sustain ~98% of the dense fp16 peak at one wave per SIMD; 16 x 16 x 32 ones need
// 16 chains per wave at many waves per SIMD to pass ~55%.
static_assert(kGemmMF % 2 == 0 && kGemmNF % 2 == 0, "32 x 32 tiles need even fragment counts");
struct GemmAcc {
    float16v v[kGemmMF / 2][kGemmNF / 2];
};

// One 32-wide step (one scale block) of the wave's tile from LDS buffer buf, 32 x 32 MFMA tiles: the
// block's k range in two halves of 16, lane (l32, h) supplying 16-byte chunk 2 q + h of its row to
// MFMA q -- the same chunks on both operands.
template <int FMT>
__device__ __forceinline__ void gemm_step(GemmAcc& acc, const GemmLds& L, int buf, int wm, int wn, int lane) {
    constexpr int MF = kGemmMF / 2, NF = kGemmNF / 2;
    const int l32 = lane & 31, h = lane >> 5;
    half8 B[NF][2];
    float sc[NF];
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const int r = wn * 32 * NF + j * 32 + l32;
#pragma unroll
        for (int q = 0; q < 2; q++) B[j][q] = *reinterpret_cast<const half8*>(&L.b[buf][gemm_off(r, 2 * q + h)]);
        sc[j] = FMT == 0 ? 1.0f : L.s[buf][r];
    }
#pragma unroll
    for (int i = 0; i < MF; i++) {
        const int r = wm * 32 * MF + i * 32 + l32;
        half8 A[2];
#pragma unroll
        for (int q = 0; q < 2; q++) A[q] = *reinterpret_cast<const half8*>(&L.a[buf][gemm_off(r, 2 * q + h)]);
#pragma unroll
        for (int j = 0; j < NF; j++) {
            if constexpr (FMT == 0) {
                acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], acc.v[i][j], 0, 0, 0);
                acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], acc.v[i][j], 0, 0, 0);
            } else {
                float16v blk = {};
                blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], blk, 0, 0, 0);
                blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], blk, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; e++) acc.v[i][j][e] = __builtin_fmaf(sc[j], blk[e], acc.v[i][j][e]);
            }
        }
    }
}

// Grid: one workgroup per BM x BN output tile (1-D, remapped: each XCD -- the hardware deals
// workgroups round-robin over the 8 -- takes a contiguous range, walked in groups of 8 token tiles
// so that concurrent workgroups share activation and weight tiles in that XCD's L2).
// With partial != nullptr the grid holds `slices` workgroups per tile, each summing one slice of
// K's steps into partial[slice][t][n] (f32, row stride N); mm_splitk_reduce adds the slices and
// applies the epilogue.
template <int FMT, typename TY>
__global__ __launch_bounds__(kGemmThreads, 2) void mm_gemm_kernel(MmArgs a, int tiles_m, int tiles_n, int slices, float* partial) {
    __shared__ __align__(16) GemmLds L;
    constexpr int MF = kGemmMF, NF = kGemmNF;
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6, wm = wave % kGemmWM, wn = wave / kGemmWM;

    uint32_t b = blockIdx.x;
    const uint32_t nb = gridDim.x;
    if (nb % 8 == 0) b = (b % 8) * (nb / 8) + b / 8;
    const int slice = static_cast<int>(b % static_cast<uint32_t>(slices));
    b /= static_cast<uint32_t>(slices);
    constexpr int GM = 8;
    const int group = static_cast<int>(b) / (GM * tiles_n);
    const int first_m = group * GM, gm = min(GM, tiles_m - first_m);
    const int in_group = static_cast<int>(b) - group * GM * tiles_n;
    const int64_t m0 = static_cast<int64_t>(first_m + in_group % gm) * kGemmBM;
    const int64_t n0 = static_cast<int64_t>(in_group / gm) * kGemmBN;

    GemmAcc acc = {};

    // Two register sets alternate: each step's global pieces are requested two steps before they are
    // written to LDS (requests past the last step re-read it: in bounds, never stored), so the loads
    // have two steps of MFMAs to arrive.
    const int nk_all = a.K / kGemmBK, per = (nk_all + slices - 1) / slices;
    const int k_first = slice * per, nk = min(nk_all - k_first, per), lastk = k_first + nk - 1;
    if (nk > 0) {  // a slice past the end of K (possible only in the last tile's tail) adds zeros
        GemmRegs<FMT> r0, r1;
        gemm_load<FMT>(r0, a, m0, n0, k_first * kGemmBK, tid);
        gemm_load<FMT>(r1, a, m0, n0, min(k_first + 1, lastk) * kGemmBK, tid);
        gemm_store<FMT>(L, 0, r0, tid);
        __syncthreads();
        gemm_load<FMT>(r0, a, m0, n0, min(k_first + 2, lastk) * kGemmBK, tid);
        for (int ks = 0;; ks += 2) {
            gemm_step<FMT>(acc, L, 0, wm, wn, lane);
            if (ks + 1 >= nk) break;
            gemm_store<FMT>(L, 1, r1, tid);
            __syncthreads();
            gemm_load<FMT>(r1, a, m0, n0, min(k_first + ks + 3, lastk) * kGemmBK, tid);
            gemm_step<FMT>(acc, L, 1, wm, wn, lane);
            if (ks + 2 >= nk) break;
            gemm_store<FMT>(L, 0, r0, tid);
            __syncthreads();
            gemm_load<FMT>(r0, a, m0, n0, min(k_first + ks + 4, lastk) * kGemmBK, tid);
        }
    }
    auto put = [&](int64_t t, int64_t n, float v) {
        if (t >= a.T || n >= a.N) return;
        if (partial) partial[(static_cast<int64_t>(slice) * a.T + t) * a.N + n] = v;
        else epilogue<TY>(a, t, n, v);
    };
    // Lane (l32, h) holds C[token 8 (e / 4) + 4 h + e % 4][row l32] of each 32 x 32 tile.
    const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < NF / 2; j++)
#pragma unroll
        for (int i = 0; i < MF / 2; i++)
#pragma unroll
            for (int e = 0; e < 16; e++)
                put(m0 + wm * 16 * MF + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3), n0 + wn * 16 * NF + j * 32 + l32,
                    acc.v[i][j][e]);
}

// The sum over slices of partial[slice][t][n .. n + width), added in slice order. Eight slices'
// loads are in flight per round (one memory round trip for up to eight slices): indices past the
// last slice re-read it and are not added.
template <typename V>
__device__ __forceinline__ V sum_slices(const float* partial, int64_t total, int64_t i, int slices) {
    V v = *reinterpret_cast<const V*>(partial + i);
    for (int s0 = 0; s0 < slices; s0 += 8) {
        V p[8];
#pragma unroll
        for (int q = 0; q < 8; q++)
            p[q] = *reinterpret_cast<const V*>(partial + static_cast<int64_t>(min(s0 + q, slices - 1)) * total + i);
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (s0 + q > 0 && s0 + q < slices) v += p[q];
    }
    return v;
}

// y = epilogue(sum over slices of partial[slice][t][n]), slices added in order.
template <typename TY>
__global__ __launch_bounds__(256) void mm_splitk_reduce(MmArgs a, const float* partial, int slices) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = a.T * static_cast<int64_t>(a.N);
    if (i >= total) return;
    const float v = sum_slices<float>(partial, total, i, slices);
    const int64_t t = i / a.N, n = i - t * a.N;
    epilogue<TY>(a, t, n, v);
}

// The same, four neighbouring outputs of one token row per thread (N % 4 == 0: 16-byte loads).
template <typename TY>
__global__ __launch_bounds__(256) void mm_splitk_reduce4(MmArgs a, const float* partial, int slices) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    const int64_t total = a.T * static_cast<int64_t>(a.N);
    if (i >= total) return;
    const float4v v = sum_slices<float4v>(partial, total, i, slices);
    const int64_t t = i / a.N, n = i - t * a.N;
#pragma unroll
    for (int e = 0; e < 4; e++) epilogue<TY>(a, t, n + e, v[e]);
}

// ---------------------------------------------------------------- prefill GEMM, 64-wide stages
//
// Workgroup tiles of BM tokens x BN weight rows over WGM x WGN waves, each wave a (32 TM) x (32 TN)
// grid of v_mfma_f32_32x32x16_f16 tiles; K staged 64 at a time -- two scale blocks per LDS stage --
// with one set of prefetch registers a stage ahead (the loads have a whole stage of MFMAs to
// arrive) and double-buffered LDS (one barrier per stage). LDS rows are 64 halves padded to 72
// (144 bytes: the 16 rows a ds_read_b128 serves per pass fall on distinct 16-byte bank groups).
// Tile size sets the reuse: every stage loads (BM + BN) x 64 operands for BM x BN x 64 MACs, and at
// 128 x 128 feeding the MFMAs at full rate would take all of the L2's bandwidth (measured: the L1s
// then wait on L2 half the time). Large FP8 / FP4 problems take 256-token x 128-row tiles (one
// workgroup of eight waves per CU, 110 KB of LDS), which also decode each weight tile once per 256
// tokens: measured 10-20% faster than 128 x 128 there, and slightly slower for F16, which keeps
// 128 x 128. (256 x 256 tiles need 128 accumulators per lane besides the staging registers and
// spill at two waves per SIMD.) Needs K % 64 == 0; other K take the 32-wide kernel above.
constexpr int kG2Row = 72;  // halves per staged row: 64 plus 8 of padding
constexpr int kG2BK = 64;
constexpr int kG2Depth = 2;  // F16: stages of global prefetch in registers (the scaled formats: 1)

template <int BM_, int BN_, int WGM_, int WGN_>
struct G2Cfg {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
    static constexpr int threads = 64 * WGM * WGN;
    static constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;  // 32 x 32 tiles per wave
    static_assert(TM * 32 * WGM == BM && TN * 32 * WGN == BN, "wave tiles of whole 32 x 32 MFMA tiles");
    static_assert(BM * 8 % threads == 0 && BN * 4 % threads == 0 && BN * 2 <= threads,
                  "load split: whole pieces per thread, at most one scale per thread");
};
typedef G2Cfg<128, 128, 2, 2> G2Small;
typedef G2Cfg<256, 128, 4, 2> G2Big;

template <class C>
struct Gemm2Lds {
    half_t a[2][C::BM * kG2Row];
    half_t b[2][C::BN * kG2Row];
    float s[2][2][C::BN];  // [buffer][block of the stage][row]: f16 scale times the decode factor
};

template <int FMT, class C>
struct Gemm2Regs {
    static constexpr int NA = C::BM * 8 / C::threads;   // activation pieces (16 bytes) per thread
    static constexpr int NW = C::BN * (FMT == 0 ? 8 : 4) / C::threads;
    uint4v a[NA];
    typename VecOf<uint32_t, FMT == 2 ? 2 : 4>::V w[NW];  // F16: 8 halves; FP8: 16 codes; FP4: half a block (16 codes)
    half_t s;  // FP8 / FP4: the scale of (row tid / 2, block tid % 2), threads below 2 BN
};

// Stage k0 (a multiple of 64). Activation piece p = tid + threads i: row p / 8, 16-byte column p % 8
// (each row's 128 bytes from 8 neighbouring threads). F16 weights the same; FP8 piece p: row p / 4,
// 16 codes at byte 16 (p % 4) of the stage's 64; FP4 piece p: row p / 4, 8 bytes at byte 8 (p % 4) of
// the stage's 32 (half of block (p % 4) / 2).
template <int FMT, class C>
__device__ __forceinline__ void gemm2_load(Gemm2Regs<FMT, C>& r, const MmArgs& a, int64_t m0, int64_t n0, int k0, int tid) {
    typedef Gemm2Regs<FMT, C> R;
    const int64_t lastT = a.T - 1, lastN = a.N - 1;
#pragma unroll
    for (int i = 0; i < R::NA; i++) {
        const int p = tid + C::threads * i, row = p >> 3, c = p & 7;
        const half_t* xr = static_cast<const half_t*>(a.x) + min(m0 + row, lastT) * a.xs;
        r.a[i] = *reinterpret_cast<const uint4v*>(xr + k0 + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < R::NW; i++) {
        const int p = tid + C::threads * i;
        if constexpr (FMT == 0) {
            const int row = p >> 3, c = p & 7;
            r.w[i] = *reinterpret_cast<const uint4v*>(a.w + min(n0 + row, lastN) * a.rb + 2 * (k0 + 8 * c));
        } else if constexpr (FMT == 1) {
            const int row = p >> 2, c = p & 3;
            r.w[i] = *reinterpret_cast<const uint4v*>(a.w + min(n0 + row, lastN) * a.rb + k0 + 16 * c);
        } else {
            const int row = p >> 2, c = p & 3;
            r.w[i] = *reinterpret_cast<const uint2v*>(a.w + min(n0 + row, lastN) * a.rb + k0 / 2 + 8 * c);
        }
    }
    if (FMT != 0 && (C::BN * 2 == C::threads || tid < C::BN * 2)) {
        const int row = tid >> 1, bb = tid & 1;
        const uint8_t* sr = a.w + min(n0 + row, lastN) * a.rb + (FMT == 1 ? a.K : a.K / 2);
        r.s = *reinterpret_cast<const half_t*>(sr + 2 * (k0 / kBlockK + bb));
    }
}

// FP4 byte SEL of word q -> its two weights as f16 (low nibble first); SEL must be a literal.
#define NEKO_FP4_PAIR(q, SEL) __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4((q), 1.0f, SEL))

template <int FMT, class C>
__device__ __forceinline__ void gemm2_store(Gemm2Lds<C>& L, int buf, const Gemm2Regs<FMT, C>& r, int tid) {
    typedef Gemm2Regs<FMT, C> R;
#pragma unroll
    for (int i = 0; i < R::NA; i++) {
        const int p = tid + C::threads * i, row = p >> 3, c = p & 7;
        *reinterpret_cast<uint4v*>(&L.a[buf][row * kG2Row + 8 * c]) = r.a[i];
    }
#pragma unroll
    for (int i = 0; i < R::NW; i++) {
        const int p = tid + C::threads * i;
        if constexpr (FMT == 0) {
            const int row = p >> 3, c = p & 7;
            *reinterpret_cast<uint4v*>(&L.b[buf][row * kG2Row + 8 * c]) = r.w[i];
        } else if constexpr (FMT == 1) {
            const int row = p >> 2, c = p & 3;  // 16 codes -> halves 16 c .. 16 c + 15
            uint32_t o[8];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t q = r.w[i][w];
                o[2 * w] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q, 0x0C010C00u));
                o[2 * w + 1] = fp8_pair_bits(__builtin_amdgcn_perm(0u, q, 0x0C030C02u));
            }
            half_t* dst = &L.b[buf][row * kG2Row + 16 * c];
            *reinterpret_cast<uint4v*>(dst) = uint4v{o[0], o[1], o[2], o[3]};
            *reinterpret_cast<uint4v*>(dst + 8) = uint4v{o[4], o[5], o[6], o[7]};
        } else {
            // Bytes 8 u .. 8 u + 7 of block v (c = 2 v + u): byte j holds weights j (low nibble) and
            // 16 + j (high nibble); the conversion yields those pairs, regrouped into natural order at
            // halves 32 v + 8 u (low) and 32 v + 16 + 8 u (high).
            const int row = p >> 2, c = p & 3, v = c >> 1, u = c & 1;
            uint32_t pr[8];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t q = r.w[i][w];
                pr[4 * w] = NEKO_FP4_PAIR(q, 0);
                pr[4 * w + 1] = NEKO_FP4_PAIR(q, 1);
                pr[4 * w + 2] = NEKO_FP4_PAIR(q, 2);
                pr[4 * w + 3] = NEKO_FP4_PAIR(q, 3);
            }
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                lo[j] = __builtin_amdgcn_perm(pr[2 * j + 1], pr[2 * j], 0x05040100u);
                hi[j] = __builtin_amdgcn_perm(pr[2 * j + 1], pr[2 * j], 0x07060302u);
            }
            half_t* dst = &L.b[buf][row * kG2Row + 32 * v + 8 * u];
            *reinterpret_cast<uint4v*>(dst) = uint4v{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<uint4v*>(dst + 16) = uint4v{hi[0], hi[1], hi[2], hi[3]};
        }
    }
    if (FMT != 0 && (C::BN * 2 == C::threads || tid < C::BN * 2))
        L.s[buf][tid & 1][tid >> 1] = static_cast<float>(r.s) * block_scale_factor<FMT>();
}
#undef NEKO_FP4_PAIR

template <class C>
struct Gemm2Acc {
    float16v v[C::TM][C::TN];
};

// The stage in LDS buffer buf: for each of its two blocks, lane (l32, h) reads 16-byte chunk
// 4 bb + 2 q + h of its rows for MFMA q -- the same chunks on both operands.
template <int FMT, class C>
__device__ __forceinline__ void gemm2_step(Gemm2Acc<C>& acc, const Gemm2Lds<C>& L, int buf, int wm, int wn, int lane) {
    constexpr int TM = C::TM, TN = C::TN;
    const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int bb = 0; bb < 2; bb++) {
        half8 B[TN][2];
        float sc[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int r = wn * 32 * TN + j * 32 + l32;
#pragma unroll
            for (int q = 0; q < 2; q++)
                B[j][q] = *reinterpret_cast<const half8*>(&L.b[buf][r * kG2Row + 8 * (4 * bb + 2 * q + h)]);
            sc[j] = FMT == 0 ? 1.0f : L.s[buf][bb][r];
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int r = wm * 32 * TM + i * 32 + l32;
            half8 A[2];
#pragma unroll
            for (int q = 0; q < 2; q++)
                A[q] = *reinterpret_cast<const half8*>(&L.a[buf][r * kG2Row + 8 * (4 * bb + 2 * q + h)]);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (FMT == 0) {
                    acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], acc.v[i][j], 0, 0, 0);
                    acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], acc.v[i][j], 0, 0, 0);
                } else {
                    float16v blk = {};
                    blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0], B[j][0], blk, 0, 0, 0);
                    blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[1], B[j][1], blk, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; e++) acc.v[i][j][e] = __builtin_fmaf(sc[j], blk[e], acc.v[i][j][e]);
                }
            }
        }
    }
}

// Grid and split of K as mm_gemm_kernel (tiles of BM x BN), in stages of 64.
template <int FMT, typename TY, class C>
__global__ __launch_bounds__(C::threads, 2) void mm_gemm2_kernel(MmArgs a, int tiles_m, int tiles_n, int slices, float* partial) {
    static_assert(sizeof(Gemm2Lds<C>) >= (C::threads / 64) * kTileLdsFloats * sizeof(float), "epilogue scratch");
    extern __shared__ __align__(16) uint8_t g2_lds[];
    Gemm2Lds<C>& L = *reinterpret_cast<Gemm2Lds<C>*>(g2_lds);
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6, wm = wave % C::WGM, wn = wave / C::WGM;

    uint32_t b = blockIdx.x;
    const uint32_t nb = gridDim.x;
    if (nb % 8 == 0) b = (b % 8) * (nb / 8) + b / 8;
    const int slice = static_cast<int>(b % static_cast<uint32_t>(slices));
    b /= static_cast<uint32_t>(slices);
    constexpr int GM = 8;
    const int group = static_cast<int>(b) / (GM * tiles_n);
    const int first_m = group * GM, gm = min(GM, tiles_m - first_m);
    const int in_group = static_cast<int>(b) - group * GM * tiles_n;
    const int64_t m0 = static_cast<int64_t>(first_m + in_group % gm) * C::BM;
    const int64_t n0 = static_cast<int64_t>(in_group / gm) * C::BN;

    Gemm2Acc<C> acc = {};
    const int nk_all = a.K / kG2BK, per = (nk_all + slices - 1) / slices;
    const int k_first = slice * per, nk = min(nk_all - k_first, per), lastk = k_first + nk - 1;
    constexpr int depth = FMT == 0 ? kG2Depth : 1;  // the scaled formats have no registers for a second set
    if (nk > 0 && depth == 1) {
        Gemm2Regs<FMT, C> r;
        gemm2_load<FMT, C>(r, a, m0, n0, k_first * kG2BK, tid);
        gemm2_store<FMT, C>(L, 0, r, tid);
        __syncthreads();
        gemm2_load<FMT, C>(r, a, m0, n0, min(k_first + 1, lastk) * kG2BK, tid);
        for (int s = 0;; s++) {
            gemm2_step<FMT, C>(acc, L, s & 1, wm, wn, lane);
            if (s + 1 >= nk) break;
            gemm2_store<FMT, C>(L, (s + 1) & 1, r, tid);
            __syncthreads();
            gemm2_load<FMT, C>(r, a, m0, n0, min(k_first + s + 2, lastk) * kG2BK, tid);
        }
    } else if (nk > 0) {
        // Two register sets alternate, each stage's loads requested two stages before they are
        // stored (requests past the last stage re-read it: in bounds, never stored).
        Gemm2Regs<FMT, C> r0, r1;
        gemm2_load<FMT, C>(r0, a, m0, n0, k_first * kG2BK, tid);
        gemm2_load<FMT, C>(r1, a, m0, n0, min(k_first + 1, lastk) * kG2BK, tid);
        gemm2_store<FMT, C>(L, 0, r0, tid);
        __syncthreads();
        gemm2_load<FMT, C>(r0, a, m0, n0, min(k_first + 2, lastk) * kG2BK, tid);
        for (int s = 0;; s += 2) {
            gemm2_step<FMT, C>(acc, L, 0, wm, wn, lane);
            if (s + 1 >= nk) break;
            gemm2_store<FMT, C>(L, 1, r1, tid);
            __syncthreads();
            gemm2_load<FMT, C>(r1, a, m0, n0, min(k_first + s + 3, lastk) * kG2BK, tid);
            gemm2_step<FMT, C>(acc, L, 1, wm, wn, lane);
            if (s + 2 >= nk) break;
            gemm2_store<FMT, C>(L, 0, r0, tid);
            __syncthreads();
            gemm2_load<FMT, C>(r0, a, m0, n0, min(k_first + s + 4, lastk) * kG2BK, tid);
        }
    }
    // Lane (l32, h) holds C[token 8 (e / 4) + 4 h + e % 4][row l32] of each 32 x 32 tile.
    if (!partial) {
        // The operand buffers are free once every wave is past its last stage.
        __syncthreads();
        store_tiles<TY, C::TM, C::TN>(a, acc.v, reinterpret_cast<float*>(g2_lds) + wave * kTileLdsFloats,
                                      m0 + wm * 32 * C::TM, n0 + wn * 32 * C::TN, lane);
        return;
    }
    const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const int64_t n = n0 + wn * 32 * C::TN + j * 32 + l32;
        if (n >= a.N) continue;
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const float16v v = acc.v[i][j];
            unrolled<16>([&](auto ec) {
                constexpr int e = decltype(ec)::value;
                const int64_t t = m0 + wm * 32 * C::TM + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (t < a.T) partial[(static_cast<int64_t>(slice) * a.T + t) * a.N + n] = v[e];
            });
        }
    }
}

template <int FMT, typename TY, class C>
int launch_gemm2(neko_hip_ctx* ctx, dim3 grid, const MmArgs& a, int tm, int tn, int slices, float* partial) {
    constexpr size_t lds = sizeof(Gemm2Lds<C>);
    static std::atomic<uint64_t> allowed{0};
    if (int rc = allow_lds(ctx, reinterpret_cast<const void*>(&mm_gemm2_kernel<FMT, TY, C>), lds, allowed)) return rc;
    hipLaunchKernelGGL((mm_gemm2_kernel<FMT, TY, C>), grid, dim3(C::threads), lds, ctx->stream, a, tm, tn, slices, partial);
    return NEKO_OK;
}

template <class C>
int launch_gemm2_fmt(neko_hip_ctx* ctx, int fmt, int y_dtype, dim3 grid, const MmArgs& a, int tm, int tn, int slices,
                     float* partial) {
    const bool f16 = y_dtype == NEKO_DT_F16;
    switch (fmt) {
        case NEKO_FMT_F16:
            if constexpr (C::BM == G2Small::BM)
                return f16 ? launch_gemm2<0, half_t, C>(ctx, grid, a, tm, tn, slices, partial)
                           : launch_gemm2<0, float, C>(ctx, grid, a, tm, tn, slices, partial);
            else
                return fail(ctx, NEKO_ERR_INVALID, "matmul: F16 rows take the 128 x 128 tiles");
        case NEKO_FMT_FP8:
            return f16 ? launch_gemm2<1, half_t, C>(ctx, grid, a, tm, tn, slices, partial)
                       : launch_gemm2<1, float, C>(ctx, grid, a, tm, tn, slices, partial);
        default:
            return f16 ? launch_gemm2<2, half_t, C>(ctx, grid, a, tm, tn, slices, partial)
                       : launch_gemm2<2, float, C>(ctx, grid, a, tm, tn, slices, partial);
    }
}

// ---------------------------------------------------------------- generic path

// W[row][k] as f32, exact: the code's f16 pattern widened, times 2^8 / 2^14, times the f16 scale.
__device__ __forceinline__ float weight_at(int fmt, const uint8_t* row, int K, int k) {
    if (fmt == NEKO_FMT_F16) return static_cast<float>(reinterpret_cast<const half_t*>(row)[k]);
    const int b = k / kBlockK;
    if (fmt == NEKO_FMT_FP8) {
        const uint32_t c = row[k];
        const half_t s = *reinterpret_cast<const half_t*>(row + K + 2 * b);
        const uint16_t h = static_cast<uint16_t>(((c & 0x7Fu) << 7) | ((c & 0x80u) << 8));
        return static_cast<float>(__builtin_bit_cast(half_t, h)) * (static_cast<float>(s) * 256.0f);
    }
    const int j = k % kBlockK;
    const uint32_t byte = row[b * (kBlockK / 2) + (j & 15)];
    const uint32_t c = j < 16 ? (byte & 0xFu) : (byte >> 4);
    const half_t s = *reinterpret_cast<const half_t*>(row + K / 2 + 2 * b);
    const uint16_t h = static_cast<uint16_t>(((c & 7u) << 9) | ((c & 8u) << 12));
    return static_cast<float>(__builtin_bit_cast(half_t, h)) * (static_cast<float>(s) * 16384.0f);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// ---------------------------------------------------------------- f32 activations on the MFMA kernels
//
// Row t of f32 activations becomes two f16 rows, scaled by a power of two s_t that puts the row's
// largest finite magnitude in [2^14, 2^15): hi = f16(x s_t), lo = f16(x s_t - hi). hi + lo holds x s_t
// to within 2^-22 of its magnitude (the largest |x| never overflows f16, values more than 2^28 below
// it lose bits only beside it), so y = (hi . W + lo . W) / s_t, two f16 matmuls and an exact rescale,
// stays far inside the f32 summation bound that every matmul path meets. An infinite or NaN value
// keeps its value in hi (inf * s_t = inf) with lo = 0, so its outputs are the +-inf / NaN the f32 dot
// product gives, and the row's finite values keep their scale.
constexpr int kSplitThreads = 256;

// One workgroup per row: the row's largest finite magnitude, then its two planes and 1 / s_t.
__global__ __launch_bounds__(kSplitThreads) void split_rows_kernel(const float* x, int64_t xs, int K, half_t* hi,
                                                                   half_t* lo, float* inv_s) {
    __shared__ float part[kSplitThreads / kWave];
    const int tid = static_cast<int>(threadIdx.x);
    const int64_t t = blockIdx.x;
    const float4v* xr = reinterpret_cast<const float4v*>(x + t * xs);
    const int K4 = K / 4;
    float m = 0.0f;
    for (int i = tid; i < K4; i += kSplitThreads) {
        const float4v v = xr[i];
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (fabsf(v[e]) <= 3.4028235e38f) m = fmaxf(m, fabsf(v[e]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) part[tid >> 6] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kSplitThreads / kWave; w++) m = fmaxf(m, part[w]);
    int e = 0;
    if (m > 0.0f && m <= 3.4028235e38f) (void)frexpf(m, &e);  // m in [2^(e-1), 2^e)
    const int sh = max(-126, min(126, 15 - e));                  // m * 2^sh in [2^14, 2^15)
    const float sc = ldexpf(1.0f, sh);
    if (tid == 0) inv_s[t] = ldexpf(1.0f, -sh);
    half_t* h = hi + t * K;
    half_t* l = lo + t * K;
    for (int i = tid; i < K4; i += kSplitThreads) {
        const float4v v = xr[i];
        half4 vh, vl;
#pragma unroll
        for (int e2 = 0; e2 < 4; e2++) {
            const float u = v[e2] * sc;
            vh[e2] = f16_rne(u);
            vl[e2] = fabsf(u) <= 3.4028235e38f ? f16_rne(u - static_cast<float>(vh[e2])) : half_t(0.0f);
        }
        reinterpret_cast<half4*>(h)[i] = vh;
        reinterpret_cast<half4*>(l)[i] = vl;
    }
}

// y[t][n] = epilogue(sums[t][n] / s_t): the row's scale undone (exact), then bias, GELU, accumulate.
template <typename TY>
__global__ __launch_bounds__(256) void combine_rows_kernel(MmArgs a, const float* sums, const float* inv_s) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.T * a.N) return;
    const int64_t t = i / a.N, n = i - t * a.N;
    epilogue<TY>(a, t, n, sums[i] * inv_s[t]);
}

// Grid: x = weight rows, y = groups of 4 tokens; one wave each.
template <typename TX, typename TY>
__global__ __launch_bounds__(64) void mm_generic_kernel(MmArgs a) {
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t n = blockIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * 4;
    const int nt = static_cast<int>(min(static_cast<int64_t>(4), a.T - t0));
    const uint8_t* row = a.w + n * a.rb;
    const TX* x = static_cast<const TX*>(a.x) + t0 * a.xs;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = lane; k < a.K; k += kWave) {
        const float wk = weight_at(a.fmt, row, a.K, k);
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (j < nt) acc[j] += to_f32(x[j * a.xs + k]) * wk;
    }
    float mine = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float s = wave_sum_f32(acc[j]);
        if (lane == j) mine = s;
    }
    if (lane < nt) epilogue<TY>(a, t0 + lane, n, mine);
}

// ---------------------------------------------------------------- launch

template <int FMT, int NT, typename TX>
int launch_gemv(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, int kw) {
    const size_t lds = gemv_lds_bytes(a.K, NT, static_cast<int>(sizeof(TX)));
    if (y_dtype == NEKO_DT_F16)
        hipLaunchKernelGGL((mm_gemv_kernel<FMT, NT, half_t, TX>), grid, dim3(64 * kGemvWaves), lds, ctx->stream, a, kw);
    else
        hipLaunchKernelGGL((mm_gemv_kernel<FMT, NT, float, TX>), grid, dim3(64 * kGemvWaves), lds, ctx->stream, a, kw);
    return after_launch(ctx, "neko_hip_matmul");
}

template <int FMT>
int launch_gemv_nt(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, int kw, int nt, bool x_f32) {
    if (x_f32) {  // f32 activations: 1, 2 or 4 tokens per pass
        switch (nt) {
            case 1: return launch_gemv<FMT, 1, float>(ctx, a, y_dtype, grid, kw);
            case 2: return launch_gemv<FMT, 2, float>(ctx, a, y_dtype, grid, kw);
            default: return launch_gemv<FMT, 4, float>(ctx, a, y_dtype, grid, kw);
        }
    }
    switch (nt) {
        case 1: return launch_gemv<FMT, 1, half_t>(ctx, a, y_dtype, grid, kw);
        default:  // 2, or 4 where the GEMV takes more than two tokens
            if constexpr (kGemvMaxT > 2) {
                if (nt == 4) return launch_gemv<FMT, 4, half_t>(ctx, a, y_dtype, grid, kw);
            }
            return launch_gemv<FMT, 2, half_t>(ctx, a, y_dtype, grid, kw);
    }
}

template <int FMT, int TT>
int launch_tile(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, int waves) {
    const size_t lds = tile_lds_bytes(FMT, waves, TT);
    if (y_dtype == NEKO_DT_F16)
        hipLaunchKernelGGL((mm_tile_kernel<FMT, TT, half_t>), grid, dim3(64 * waves), lds, ctx->stream, a);
    else
        hipLaunchKernelGGL((mm_tile_kernel<FMT, TT, float>), grid, dim3(64 * waves), lds, ctx->stream, a);
    return after_launch(ctx, "neko_hip_matmul");
}

template <int FMT>
int launch_tile_tt(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, int waves, int tt) {
    switch (tt) {
        case 1: return launch_tile<FMT, 1>(ctx, a, y_dtype, grid, waves);
        case 2: return launch_tile<FMT, 2>(ctx, a, y_dtype, grid, waves);
        case 3: return launch_tile<FMT, 3>(ctx, a, y_dtype, grid, waves);
        default: return launch_tile<FMT, 4>(ctx, a, y_dtype, grid, waves);
    }
}

template <int FMT, int TT>
int launch_tile2(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, size_t lds, int slice_blocks, float* partial) {
    const int nblk = static_cast<int>(a.K / kBlockK);
    const int last_blocks = nblk - (static_cast<int>(grid.z) - 1) * slice_blocks;
    const FastDiv full = make_fast_div(static_cast<uint32_t>(4 * slice_blocks));
    const FastDiv last = make_fast_div(static_cast<uint32_t>(4 * last_blocks));
    if (y_dtype == NEKO_DT_F16)
        hipLaunchKernelGGL((mm_tile2_kernel<FMT, TT, half_t>), grid, dim3(64 * kT2Waves), lds, ctx->stream, a, slice_blocks,
                           partial, full, last);
    else
        hipLaunchKernelGGL((mm_tile2_kernel<FMT, TT, float>), grid, dim3(64 * kT2Waves), lds, ctx->stream, a, slice_blocks,
                           partial, full, last);
    return after_launch(ctx, "neko_hip_matmul");
}

template <int FMT>
int launch_tile2_tt(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, dim3 grid, size_t lds, int slice_blocks, float* partial, int tt) {
    switch (tt) {
        case 1: return launch_tile2<FMT, 1>(ctx, a, y_dtype, grid, lds, slice_blocks, partial);
        case 2: return launch_tile2<FMT, 2>(ctx, a, y_dtype, grid, lds, slice_blocks, partial);
        default:  // tt 3, or 4 where the kernel takes more than 48 tokens
            if constexpr (kT2MaxT > 49) {
                if (tt == 4) return launch_tile2<FMT, 4>(ctx, a, y_dtype, grid, lds, slice_blocks, partial);
            }
            return launch_tile2<FMT, 3>(ctx, a, y_dtype, grid, lds, slice_blocks, partial);
    }
}

// y = epilogue(partial slices added in order), after a split-K launch.
int launch_splitk_reduce(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, const float* partial, int slices, const char* what) {
    const int64_t total = a.T * a.N;
    const bool vec = a.N % 4 == 0;
    const int64_t blocks = (total + (vec ? 1023 : 255)) / (vec ? 1024 : 256);
    NEKO_REQUIRE(ctx, blocks <= 0x7fffffff, "%s: output too large", what);
    const dim3 grid(static_cast<uint32_t>(blocks));
    if (vec) {
        if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_splitk_reduce4<half_t>), grid, dim3(256), 0, ctx->stream, a, partial, slices);
        else hipLaunchKernelGGL((mm_splitk_reduce4<float>), grid, dim3(256), 0, ctx->stream, a, partial, slices);
    } else {
        if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_splitk_reduce<half_t>), grid, dim3(256), 0, ctx->stream, a, partial, slices);
        else hipLaunchKernelGGL((mm_splitk_reduce<float>), grid, dim3(256), 0, ctx->stream, a, partial, slices);
    }
    return after_launch(ctx, what);
}

// The scratch memory of neko_hip_matmul_noalloc: split-K partial sums, and for f32 activations the
// two f16 planes and their sums, in a fixed array in device memory, so that entry point never
// allocates. Each device holds its own copy (the runtime places it when the code object loads there)
// until the process ends. 32 MiB covers every split the planner below makes for the Qwen3-0.6B/4B
// layer projections at any token count with f16 activations (at most 30 MiB); requests beyond it are
// rejected.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device address of `scratch` per device ordinal, looked up once per device by matmul_scratch_setup,
// and the context that may use it: the first to call neko_hip_matmul_noalloc on the device, until it
// is destroyed. On the host, `scratch` names a host-side stand-in, never the device array: only these
// addresses reach kernels.
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;
std::map<int, const neko_hip_ctx*> g_scratch_owner;

// Device memory a call may use instead of the context's workspace: p == nullptr means the workspace
// (which grows); otherwise `bytes` at p and no more.
struct Fixed {
    uint8_t* p = nullptr;
    size_t bytes = 0;
};

// Where split-K partials go: the context's growable workspace, or the fixed memory, never grown.
int partial_buffer(neko_hip_ctx* ctx, const Fixed& fixed, size_t bytes, float** out, const char* what) {
    if (fixed.p) {
        if (bytes > fixed.bytes)
            return fail(ctx, NEKO_ERR_UNSUPPORTED,
                        "%s: this shape splits K into %zu bytes of partial sums; the allocation-free entry point "
                        "has %zu of its %zu bytes for them (call neko_hip_matmul instead)",
                        what, bytes, fixed.bytes, kScratchBytes);
        *out = reinterpret_cast<float*>(fixed.p);
        return NEKO_OK;
    }
    void* ws = nullptr;
    if (int rc = workspace(ctx, bytes, &ws)) return rc;
    *out = static_cast<float*>(ws);
    return NEKO_OK;
}

int matmul_impl(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w, int64_t row_bytes,
                int fmt, int64_t N, const float* bias, void* y, int64_t y_stride, int flags, int x_dtype, int y_dtype,
                const Fixed& fixed, const char* what);

// From this many tokens, f32 activations go through the MFMA kernels as two f16 planes. Measured on
// the Qwen3-4B projections: at 3-8 tokens the f32 GEMV is faster in every format but one case (F16
// down at 6 tokens, 5% slower; FP4 gate/up at 5-8 tokens 30-31 us against 36-38, FP4 down 23-25
// against 36-37); at 10-16 the planes win for gate/up (16 tokens: 41-53 us against 52-68) and the
// F16 / FP8 down, the GEMV for q/k/v and the FP4 down; at 512 tokens the planes are 16x faster.
// Weights of at most kF32SmallNK elements keep the GEMV through 16 tokens: at 10-16 it measured
// 1.1-2.2x faster than the planes for the Qwen3-4B q/k/v [6144, 2560] and o [2560, 4096] and the
// Qwen3-0.6B projections (the planes' four launches dominate there).
constexpr int64_t kF32SplitMinT = 9;
// From this many tokens the plain F16 product (f16 activations) goes to hipBLASLt (matmul_lib.hip):
// measured faster than the own GEMM kernels on every Qwen3-4B projection from 512 tokens (12-40%); at
// 64-256 tokens only for the widest (gate/up, 19456 rows: 17-31%), while the own kernels win for the
// 2560-row projections (down by up to 43%) -- hence from kLibMinTWide tokens for kLibWideN rows.
constexpr int64_t kLibMinT = 512;
constexpr int64_t kLibMinTWide = 64;
constexpr int64_t kLibWideN = 16384;
constexpr int64_t kF32SplitMinTSmall = 17;
constexpr int64_t kF32SmallNK = int64_t{1} << 24;

// f32 activations (16-byte aligned rows, K % 32 == 0) as two f16 planes: both through the f16 paths
// into f32 sums in workspace slot 1 (any split of K uses slot 0), then rescaled into y with the call's
// bias / GELU / accumulate. With fixed memory, the planes and sums take its start and any split of K
// the rest.
int matmul_f32_split(neko_hip_ctx* ctx, const MmArgs& a, int y_dtype, const Fixed& fixed, const char* what) {
    const int64_t T = a.T, K = a.K, N = a.N;
    const auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
    const size_t plane = up(static_cast<size_t>(T) * K * 2), sums = up(static_cast<size_t>(T) * N * 4);
    const size_t need = 2 * plane + sums + up(static_cast<size_t>(T) * 4);
    uint8_t* base = nullptr;
    Fixed rest;
    if (fixed.p) {
        if (need > fixed.bytes)
            return fail(ctx, NEKO_ERR_UNSUPPORTED,
                        "%s: f32 activations of this shape need %zu bytes for their f16 planes and sums; the "
                        "allocation-free entry point holds at most %zu (call neko_hip_matmul instead)",
                        what, need, fixed.bytes);
        base = fixed.p;
        rest.p = fixed.p + need;
        rest.bytes = fixed.bytes - need;
    } else {
        void* ws = nullptr;
        if (int rc = workspace(ctx, need, &ws, 1)) return rc;
        base = static_cast<uint8_t*>(ws);
    }
    half_t* hi = reinterpret_cast<half_t*>(base);
    half_t* lo = reinterpret_cast<half_t*>(base + plane);
    float* s = reinterpret_cast<float*>(base + 2 * plane);
    float* inv = reinterpret_cast<float*>(base + 2 * plane + sums);
    NEKO_REQUIRE(ctx, T <= 0x7fffffff && T * N / 256 < 0x7fffffff, "%s: T=%lld too large", what, (long long)T);
    hipLaunchKernelGGL(split_rows_kernel, dim3(static_cast<uint32_t>(T)), dim3(kSplitThreads), 0, ctx->stream,
                       static_cast<const float*>(a.x), a.xs, static_cast<int>(K), hi, lo, inv);
    if (int rc = after_launch(ctx, what)) return rc;
    if (int rc = matmul_impl(ctx, hi, K, T, K, a.w, a.rb, a.fmt, N, nullptr, s, N, 0, NEKO_DT_F16, NEKO_DT_F32, rest, what))
        return rc;
    if (int rc = matmul_impl(ctx, lo, K, T, K, a.w, a.rb, a.fmt, N, nullptr, s, N, kAccumulate, NEKO_DT_F16, NEKO_DT_F32,
                             rest, what))
        return rc;
    const dim3 grid(static_cast<uint32_t>((T * N + 255) / 256));
    if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((combine_rows_kernel<half_t>), grid, dim3(256), 0, ctx->stream, a, s, inv);
    else hipLaunchKernelGGL((combine_rows_kernel<float>), grid, dim3(256), 0, ctx->stream, a, s, inv);
    return after_launch(ctx, what);
}

int matmul_impl(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w, int64_t row_bytes,
                int fmt, int64_t N, const float* bias, void* y, int64_t y_stride, int flags, int x_dtype, int y_dtype,
                const Fixed& fixed, const char* what) {
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(x_dtype) && valid_dtype(y_dtype), "%s: bad dtype x=%d y=%d", what, x_dtype, y_dtype);
    NEKO_REQUIRE(ctx, fmt == NEKO_FMT_F16 || fmt == NEKO_FMT_FP8 || fmt == NEKO_FMT_FP4, "%s: bad weight format %d", what,
                 fmt);
    NEKO_REQUIRE(ctx, (flags & ~(kGelu | kAccumulate)) == 0, "%s: bad flags %d", what, flags);
    NEKO_REQUIRE(ctx, T >= 0 && K > 0 && N >= 0 && K <= (1 << 30) && N <= (1 << 30),
                 "%s: bad shape T=%lld K=%lld N=%lld", what, (long long)T, (long long)K, (long long)N);
    NEKO_REQUIRE(ctx, fmt == NEKO_FMT_F16 || K % kBlockK == 0, "%s: FP8/FP4 rows need K %% 32 == 0 (K=%lld)", what,
                 (long long)K);
    NEKO_REQUIRE(ctx, row_bytes >= static_cast<int64_t>(neko_quant_row_bytes(fmt, K)) && row_bytes % 2 == 0,
                 "%s: row_bytes %lld below the %zu bytes of a K=%lld row", what, (long long)row_bytes,
                 neko_quant_row_bytes(fmt, K), (long long)K);
    NEKO_REQUIRE(ctx, x_stride >= K && y_stride >= N, "%s: strides x=%lld y=%lld below K=%lld / N=%lld", what,
                 (long long)x_stride, (long long)y_stride, (long long)K, (long long)N);
    if (T == 0 || N == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, x && w && y, "%s: null pointer", what);
    NEKO_REQUIRE(ctx, T <= INT64_MAX / x_stride && T <= INT64_MAX / y_stride, "%s: too many rows", what);
    const size_t xbytes = static_cast<size_t>((T - 1) * x_stride + K) * dtype_size(x_dtype);
    const size_t ybytes = static_cast<size_t>((T - 1) * y_stride + N) * dtype_size(y_dtype);
    const size_t wbytes = static_cast<size_t>(N) * static_cast<size_t>(row_bytes);
    NEKO_REQUIRE(ctx, !overlaps(y, ybytes, x, xbytes) && !overlaps(y, ybytes, w, wbytes),
                 "%s: y may not overlap x or the weights", what);

    MmArgs a{x, x_stride, T, static_cast<const uint8_t*>(w), row_bytes, static_cast<int>(K), static_cast<int>(N), bias,
             y, y_stride, flags, fmt, 0, aligned(y, 4 * dtype_size(y_dtype)) && y_stride % 4 == 0};
    const bool fast = x_dtype == NEKO_DT_F16 && K % kBlockK == 0 && aligned(x, 16) && x_stride % 8 == 0 &&
                      aligned(w, 16) && row_bytes % 16 == 0;
    const bool fast32 = x_dtype == NEKO_DT_F32 && K % kBlockK == 0 && aligned(x, 16) && x_stride % 4 == 0 &&
                        aligned(w, 16) && row_bytes % 16 == 0;
    // f32 activations from kF32SplitMinT tokens: two f16 planes through the MFMA kernels; below, the
    // f32 GEMV.
    if (fast32 && T >= (N * K <= kF32SmallNK ? kF32SplitMinTSmall : kF32SplitMinT))
        return matmul_f32_split(ctx, a, y_dtype, fixed, what);
    // Decode-sized T: the GEMV path, NT tokens per pass with their activations staged in 64 KB of LDS.
    int gemv_nt = 0;
    if ((fast && T <= kGemvMaxT) || (fast32 && T <= kGemv32MaxT)) {
        const int xb = fast32 ? 4 : 2;
        int nt = T <= 1 ? 1 : T <= 2 ? 2 : 4;
        while (nt > 1 && gemv_lds_bytes(static_cast<int>(K), nt, xb) > 65536) nt /= 2;
        if (gemv_lds_bytes(static_cast<int>(K), nt, xb) <= 65536) gemv_nt = nt;
    }
    if (gemv_nt > 0) {
        // kw waves share 4 rows, splitting K; a workgroup holds 8 / kw such row groups. kw: the
        // smallest power of two giving about kGemvWaveTarget waves, while every lane keeps a block.
        const int64_t chunks = (T + gemv_nt - 1) / gemv_nt;
        NEKO_REQUIRE(ctx, chunks <= 65535, "%s: T=%lld exceeds this kernel's grid", what, (long long)T);
        const int nblk = static_cast<int>(K / kBlockK);
        int kw = 1;
        while (kw < kGemvWaves && 2 * kw * 16 <= nblk &&
               (N + kGemvRows - 1) / kGemvRows * kw * chunks < kGemvWaveTarget)
            kw *= 2;
        a.blocks_per_wave = (nblk + kw - 1) / kw;
        const int64_t rows_per_wg = static_cast<int64_t>(kGemvRows) * (kGemvWaves / kw);
        const dim3 grid(static_cast<uint32_t>((N + rows_per_wg - 1) / rows_per_wg), static_cast<uint32_t>(chunks));
        switch (fmt) {
            case NEKO_FMT_F16: return launch_gemv_nt<0>(ctx, a, y_dtype, grid, kw, gemv_nt, fast32);
            case NEKO_FMT_FP8: return launch_gemv_nt<1>(ctx, a, y_dtype, grid, kw, gemv_nt, fast32);
            default: return launch_gemv_nt<2>(ctx, a, y_dtype, grid, kw, gemv_nt, fast32);
        }
    }
    // The plain F16 product at prefill sizes: hipBLASLt where the context allows it. The GELU epilogue
    // (the library has none of the reference's form), a bias added to an accumulated y (the library
    // adds y before the bias, the reference y + (dot + bias)), the allocation-free entry point (the
    // library allocates) and calls on a stream under graph capture (the library's stream-K kernels
    // clear their flags with a memset, which a captured graph does not replay reliably) stay on the own
    // kernels.
    if (fast && fmt == NEKO_FMT_F16 && (T >= kLibMinT || (T >= kLibMinTWide && N >= kLibWideN)) && ctx->use_library && !fixed.p && (flags & kGelu) == 0 &&
        !(bias && (flags & kAccumulate)) && aligned(y, 16) &&
        (y_stride * static_cast<int64_t>(dtype_size(y_dtype))) % 16 == 0) {
        bool cap = false;
        if (int rc = capturing(ctx, ctx->stream, &cap)) return rc;
        bool done = false;
        if (!cap)
            if (int rc = lt_matmul(ctx, x, x_stride, T, K, w, row_bytes, N, bias, y, y_stride, flags, y_dtype, &done))
                return rc;
        if (done) return NEKO_OK;
    }
    if (fast && T >= (fmt == NEKO_FMT_F16 ? kGemmMinTF16 : kGemmMinT)) {
        const bool v2 = K % kG2BK == 0;
        // F16: 256 x 256 tiles with direct-to-LDS loads when they give every CU at least two (with
        // fewer, the partial last round of one-per-CU workgroups cost more than the wider tiles save:
        // measured on the 2560-row projections at T = 8192, 320 tiles).
        const int64_t g3_m = (T + kG3BM - 1) / kG3BM, g3_n = (N + kG3BN - 1) / kG3BN;
        if (v2 && fmt == NEKO_FMT_F16 && g3_m * g3_n >= 2 * static_cast<int64_t>(ctx->cu_count)) {
            NEKO_REQUIRE(ctx, g3_m * g3_n <= 0x7fffffff, "%s: too many output tiles", what);
            const dim3 grid(static_cast<uint32_t>(g3_m * g3_n));
            const int tm = static_cast<int>(g3_m), tn = static_cast<int>(g3_n);
            const int rc = y_dtype == NEKO_DT_F16 ? launch_gemm3<half_t>(ctx, grid, a, tm, tn)
                                                  : launch_gemm3<float>(ctx, grid, a, tm, tn);
            if (rc) return rc;
            return after_launch(ctx, what);
        }
        if (v2 && fmt != NEKO_FMT_F16 && g3_m * g3_n >= 2 * static_cast<int64_t>(ctx->cu_count)) {
            NEKO_REQUIRE(ctx, g3_m * g3_n <= 0x7fffffff, "%s: too many output tiles", what);
            const dim3 grid(static_cast<uint32_t>(g3_m * g3_n));
            const int tm = static_cast<int>(g3_m), tn = static_cast<int>(g3_n);
            const bool h = y_dtype == NEKO_DT_F16;
            const int rc = fmt == NEKO_FMT_FP8 ? (h ? launch_gemm3q<1, half_t>(ctx, grid, a, tm, tn) : launch_gemm3q<1, float>(ctx, grid, a, tm, tn))
                                               : (h ? launch_gemm3q<2, half_t>(ctx, grid, a, tm, tn) : launch_gemm3q<2, float>(ctx, grid, a, tm, tn));
            if (rc) return rc;
            return after_launch(ctx, what);
        }
        // FP8 / FP4: 256-token x 128-row tiles (one workgroup per CU) when they alone give every CU a
        // workgroup.
        const int64_t big_m = (T + G2Big::BM - 1) / G2Big::BM, big_n = (N + G2Big::BN - 1) / G2Big::BN;
        if (v2 && fmt != NEKO_FMT_F16 && big_m * big_n >= ctx->cu_count) {
            NEKO_REQUIRE(ctx, big_m * big_n <= 0x7fffffff, "%s: too many output tiles", what);
            if (int rc = launch_gemm2_fmt<G2Big>(ctx, fmt, y_dtype, dim3(static_cast<uint32_t>(big_m * big_n)), a,
                                                 static_cast<int>(big_m), static_cast<int>(big_n), 1, nullptr))
                return rc;
            return after_launch(ctx, what);
        }
        const int64_t tiles_m = (T + kGemmBM - 1) / kGemmBM, tiles_n = (N + kGemmBN - 1) / kGemmBN;
        const int64_t tiles = tiles_m * tiles_n, nk = K / kGemmBK;
        // Split K when the tiles alone would leave CUs idle: enough slices for about two workgroups
        // per CU, each at least 8 steps long.
        int slices = 1;
        while (slices < 16 && tiles * slices * 2 <= 2 * ctx->cu_count && nk / (2 * slices) >= 8) slices *= 2;
        NEKO_REQUIRE(ctx, tiles * slices <= 0x7fffffff, "%s: too many output tiles", what);
        float* partial = nullptr;
        if (slices > 1)
            if (int rc = partial_buffer(ctx, fixed, static_cast<size_t>(slices) * T * N * sizeof(float), &partial, what))
                return rc;
        const dim3 grid(static_cast<uint32_t>(tiles * slices));
        const int tm = static_cast<int>(tiles_m), tn = static_cast<int>(tiles_n);
        if (v2) {
            if (int rc = launch_gemm2_fmt<G2Small>(ctx, fmt, y_dtype, grid, a, tm, tn, slices, partial)) return rc;
        } else if (fmt == NEKO_FMT_F16) {
            if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_gemm_kernel<0, half_t>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
            else hipLaunchKernelGGL((mm_gemm_kernel<0, float>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
        } else if (fmt == NEKO_FMT_FP8) {
            if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_gemm_kernel<1, half_t>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
            else hipLaunchKernelGGL((mm_gemm_kernel<1, float>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
        } else {
            if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_gemm_kernel<2, half_t>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
            else hipLaunchKernelGGL((mm_gemm_kernel<2, float>), grid, dim3(kGemmThreads), 0, ctx->stream, a, tm, tn, slices, partial);
        }
        if (int rc = after_launch(ctx, what)) return rc;
        if (slices > 1) return launch_splitk_reduce(ctx, a, y_dtype, partial, slices, what);
        return NEKO_OK;
    }
    // The shared-activation kernel where it measured faster than the per-wave kernel (whose single
    // launch needs no reduction of K slices): FP4 above 4 tokens, FP8 above 12, F16 above 16 (and
    // below 33, where F16 takes the GEMM).
    const bool tile2 = T < kT2MaxT && ((fmt == NEKO_FMT_FP4 && T > kT2MinFp4) || (fmt == NEKO_FMT_FP8 && T > kT2MinFp8) ||
                                       (fmt == NEKO_FMT_F16 && T > kT2MinF16));
    if (fast && tile2) {
        const int tt = static_cast<int>((T + 15) / 16);  // 1..4: one chunk of 16 tt tokens
        const int rows = static_cast<int>(T);           // token rows staged (the kernel's `rows`)
        const int64_t tiles = (N + 16 * kT2Waves - 1) / (16 * kT2Waves);
        const int nblk = static_cast<int>(K / kBlockK);
        const size_t stage = static_cast<size_t>(kT2Waves) * stage_bytes(fmt);
        // The largest slice of K whose staged activations fit beside the staging tiles; then more
        // slices (halving) until the grid holds about kT2Fill workgroups per CU, each slice at least 8
        // blocks long.
        const int cap = static_cast<int>(((kT2Lds - stage) / (2 * rows) - 8) / 32);
        int slices = (nblk + cap - 1) / cap;
        while (tiles * slices < kT2Fill * ctx->cu_count && nblk / (2 * slices) >= 8) slices *= 2;
        int slice_blocks = (nblk + slices - 1) / slices;
        slice_blocks = std::min(cap, (slice_blocks + kGroup - 1) / kGroup * kGroup);  // whole groups where possible
        slices = (nblk + slice_blocks - 1) / slice_blocks;
        NEKO_REQUIRE(ctx, tiles <= 0x7fffffff && slices <= 65535, "%s: grid too large", what);
        float* partial = nullptr;
        if (slices > 1)
            if (int rc = partial_buffer(ctx, fixed, static_cast<size_t>(slices) * T * N * sizeof(float), &partial, what))
                return rc;
        const size_t lds = t2_acts_bytes(rows, slice_blocks) + stage;
        const dim3 grid(static_cast<uint32_t>(tiles), 1u, static_cast<uint32_t>(slices));
        int rc;
        switch (fmt) {
            case NEKO_FMT_F16: rc = launch_tile2_tt<0>(ctx, a, y_dtype, grid, lds, slice_blocks, partial, tt); break;
            case NEKO_FMT_FP8: rc = launch_tile2_tt<1>(ctx, a, y_dtype, grid, lds, slice_blocks, partial, tt); break;
            default: rc = launch_tile2_tt<2>(ctx, a, y_dtype, grid, lds, slice_blocks, partial, tt); break;
        }
        if (rc || slices == 1) return rc;
        return launch_splitk_reduce(ctx, a, y_dtype, partial, slices, what);
    }
    if (fast) {
        const int tt = static_cast<int>(std::min<int64_t>(4, (T + 15) / 16));
        const int64_t chunks = (T + 16 * tt - 1) / (16 * tt);
        const int64_t tiles = (N + 15) / 16;
        NEKO_REQUIRE(ctx, chunks <= 65535, "%s: T=%lld exceeds this kernel's grid", what, (long long)T);
        // Enough waves to fill the chip, each with at least one group of K.
        const int gb = kGroup;
        const int groups = static_cast<int>((K / kBlockK + gb - 1) / gb);
        const int64_t want = (kWaveTarget + tiles * chunks - 1) / (tiles * chunks);
        int cap = std::min(kMaxWaves, max_waves(fmt, tt));
        while (cap > 1 && tile_lds_bytes(fmt, cap, tt) > 65536) cap--;
        int waves = static_cast<int>(std::min<int64_t>({cap, static_cast<int64_t>(groups), std::max<int64_t>(1, want)}));
        const int gpw = (groups + waves - 1) / waves;
        a.blocks_per_wave = gpw * gb;
        waves = (groups + gpw - 1) / gpw;
        const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(chunks));
        switch (fmt) {
            case NEKO_FMT_F16: return launch_tile_tt<0>(ctx, a, y_dtype, grid, waves, tt);
            case NEKO_FMT_FP8: return launch_tile_tt<1>(ctx, a, y_dtype, grid, waves, tt);
            default: return launch_tile_tt<2>(ctx, a, y_dtype, grid, waves, tt);
        }
    }
    const int64_t tgroups = (T + 3) / 4;
    NEKO_REQUIRE(ctx, tgroups <= 65535, "%s: T=%lld exceeds this kernel's grid", what, (long long)T);
    const dim3 grid(static_cast<uint32_t>(N), static_cast<uint32_t>(tgroups));
    if (x_dtype == NEKO_DT_F16) {
        if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_generic_kernel<half_t, half_t>), grid, dim3(64), 0, ctx->stream, a);
        else hipLaunchKernelGGL((mm_generic_kernel<half_t, float>), grid, dim3(64), 0, ctx->stream, a);
    } else {
        if (y_dtype == NEKO_DT_F16) hipLaunchKernelGGL((mm_generic_kernel<float, half_t>), grid, dim3(64), 0, ctx->stream, a);
        else hipLaunchKernelGGL((mm_generic_kernel<float, float>), grid, dim3(64), 0, ctx->stream, a);
    }
    return after_launch(ctx, what);
}

}  // namespace

void matmul_scratch_release(const neko_hip_ctx* ctx) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_owner.find(ctx->device);
    if (it != g_scratch_owner.end() && it->second == ctx) g_scratch_owner.erase(it);
}

int matmul_scratch_setup(neko_hip_ctx* ctx) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_ptr.find(ctx->device);
    if (it == g_scratch_ptr.end()) {
        void* ptr = nullptr;
        if (int rc = check(ctx, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (matmul scratch)"))
            return rc;
        it = g_scratch_ptr.emplace(ctx->device, ptr).first;
    }
    ctx->scratch = it->second;
    return NEKO_OK;
}

}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_matmul(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w,
                               int64_t row_bytes, int fmt, int64_t N, const float* bias, void* y, int64_t y_stride,
                               int flags, int x_dtype, int y_dtype) {
    return matmul_impl(ctx, x, x_stride, T, K, w, row_bytes, fmt, N, bias, y, y_stride, flags, x_dtype, y_dtype, Fixed{},
                       "neko_hip_matmul");
}

extern "C" int neko_hip_matmul_noalloc(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K,
                                       const void* w, int64_t row_bytes, int fmt, int64_t N, const float* bias, void* y,
                                       int64_t y_stride, int flags, int x_dtype, int y_dtype) {
    const char* what = "neko_hip_matmul_noalloc";
    NEKO_REQUIRE(ctx, ctx && ctx->scratch, "%s: null context, or its device's scratch address was not set up", what);
    {
        // One context per device uses the array at a time: calls through one context are ordered on
        // its stream, calls through two could overlap and overwrite each other's partial sums.
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        auto it = g_scratch_owner.find(ctx->device);
        if (it == g_scratch_owner.end()) g_scratch_owner.emplace(ctx->device, ctx);
        else if (it->second != ctx)
            return fail(ctx, NEKO_ERR_UNSUPPORTED,
                        "%s: device %d's scratch array belongs to another live context (the first to call this entry "
                        "point on the device, until it is destroyed); use that context, or neko_hip_matmul",
                        what, ctx->device);
    }
    Fixed fixed;
    fixed.p = static_cast<uint8_t*>(ctx->scratch);
    fixed.bytes = kScratchBytes;
    return matmul_impl(ctx, x, x_stride, T, K, w, row_bytes, fmt, N, bias, y, y_stride, flags, x_dtype, y_dtype, fixed,
                       what);
}
