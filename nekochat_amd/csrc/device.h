// Device helpers shared by the gfx950 kernels: 16-byte chunk types, f16/f32 conversions, and
// cross-lane reductions built from DPP (no LDS) for 64-wide wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <utility>

// The reference rounds every float product and sum separately (its portable path has no FMA), so
// kernels must not contract a*b+c into fma. The build passes -ffp-contract=off as well.
#pragma clang fp contract(off)

namespace neko_hip {

constexpr int kWave = 64;

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t uint4v __attribute__((ext_vector_type(4)));
typedef uint32_t uint2v __attribute__((ext_vector_type(2)));

// A 16-byte chunk of activations: 8 halves or 4 floats.
template <typename T>
struct Chunk16;
template <>
struct Chunk16<half_t> {
    static constexpr int N = 8;
    typedef half8 V;
};
template <>
struct Chunk16<float> {
    static constexpr int N = 4;
    typedef float4v V;
};

// Vectors of N elements of T (N * sizeof(T) in {2,4,8,16,32} bytes).
template <typename T, int N>
struct VecOf {
    typedef T V __attribute__((ext_vector_type(N)));
};
template <typename T>
struct VecOf<T, 1> {
    typedef T V;
};

template <typename V>
__device__ __forceinline__ V load_nt(const V* p) {
    return __builtin_nontemporal_load(p);
}
template <typename V>
__device__ __forceinline__ void store_nt(V* p, V v) {
    __builtin_nontemporal_store(v, p);
}

// ---------------------------------------------------------------- range-checked buffer access
// A raw buffer resource over [p, p + bytes) (stride 0; gfx9 descriptor word 3). Loads through it past
// `bytes` return zeros and stores past it are dropped by the hardware, so a wave can move a row whose
// tail covers only some lanes without a per-lane branch. That matters for the memory counter: the
// compiler's s_waitcnt placement can only count loads that every path issues, so a load under a
// branch in a loop makes the next wait drain every outstanding load and store (prefetch included).
typedef __amdgpu_buffer_rsrc_t BufRes;
__device__ __forceinline__ BufRes buf_res(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
// 16 bytes at byte offset `off`; NT sets the non-temporal cache policy (aux bit 1 on gfx94x/gfx950).
template <bool NT, typename V>
__device__ __forceinline__ V buf_load16(BufRes r, uint32_t off) {
    static_assert(sizeof(V) == 16, "16-byte vector");
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, NT ? 2 : 0));
}
// 4, 8 or 16 bytes at byte offset `off` (plain cache policy).
template <typename V>
__device__ __forceinline__ V buf_load(BufRes r, uint32_t off) {
    if constexpr (sizeof(V) == 16) return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    else if constexpr (sizeof(V) == 8) return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    else {
        static_assert(sizeof(V) == 4, "4, 8 or 16 bytes");
        return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    }
}
template <bool NT, typename V>
__device__ __forceinline__ void buf_store16(BufRes r, uint32_t off, V v) {
    static_assert(sizeof(V) == 16, "16-byte vector");
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uint4v, v), r, off, 0, NT ? 2 : 0);
}

// silu(g) = g / (1 + exp(-g)) in float, the reference's formula (cpu_ops.cpp:526-533,
// granite_model.cpp:21), with a cheaper evaluation than libm expf + IEEE division (those cost ~33
// VALU ops per element and left streaming kernels VALU-bound on MI355X; this form takes ~17):
//   exp(-g) = 2^(h + l) with h = -g*log2(e) rounded and l its exact rounding error (fma) plus the
//   low part of log2(e), evaluated as v_exp_f32(h) * (1 + l*ln2);
//   q = g / d by v_rcp_f32 and one Newton correction of the quotient, fma(fma(-q, d, g), r, q).
// The exponent argument is clamped at 126 so d stays finite (no 0 * inf in the correction); gates
// below about -87.3 then give a value of magnitude < 2^-119 instead of the reference's (also tiny
// or -0) quotient, which rounds to the same signed zero once multiplied by an fp16 operand. A +inf
// gate passes through as +inf, a zero gate keeps its sign (the correction step would turn -0 into
// +0), and -inf / NaN give NaN, as in the reference. Measured against the
// oracle over every fp16 gate value: SwiGLU outputs within 1 fp16 ulp.
__device__ __forceinline__ float silu_fast(float gate) {
    const float kLog2e = 1.44269504088896341f, kLog2eLo = 1.925963033500011e-08f, kLn2 = 0.69314718055994531f;
    const float h = gate * -kLog2e;
    const float l = __builtin_fmaf(gate, -kLog2e, -h) - gate * kLog2eLo;
    const float e = __builtin_amdgcn_exp2f(fminf(h, 126.0f)) * __builtin_fmaf(l, kLn2, 1.0f);
    const float d = 1.0f + e;
    const float r = __builtin_amdgcn_rcpf(d);
    const float q0 = gate * r;
    float q = __builtin_fmaf(__builtin_fmaf(-q0, d, gate), r, q0);
    if (gate == __builtin_inff() || gate == 0.0f) q = gate;  // +inf, and the sign of a zero gate
    return q;
}

// float(1 / sqrt(d)) of a double d, the norm scale the reference computes with a correctly rounded
// double sqrt and division before rounding to float (cpu_ops.cpp:508). Here: v_rsq_f64 and two
// Newton steps y *= 1.5 - (d/2) y^2 (about 12 double ops instead of ~40). Each step squares the
// relative error, so the double result is within a few ulps of 1/sqrt(d), and its rounding to float
// equals the reference's unless 1/sqrt(d) lies within ~2^-50 (relative) of a float rounding
// boundary, where the two may differ by one float ulp. d outside [2^-1000, 2^1000] (zero,
// subnormal, infinite or NaN) takes the exact expression.
__device__ __forceinline__ float rsqrt_to_float(double d) {
    if (!(d >= 0x1p-1000 && d <= 0x1p1000)) return static_cast<float>(1.0 / sqrt(d));
    const double h = 0.5 * d;
    double y = __builtin_amdgcn_rsq(d);
    y = y * __builtin_fma(-h * y, y, 1.5);
    y = y * __builtin_fma(-h * y, y, 1.5);
    return static_cast<float>(y);
}

// silu(g) = g * rcp(1 + 2^(-g*log2(e))): five VALU ops. Relative error vs the exact quotient is
// below |g| * 2^-24 * ln 2 (the rounding of the exponent argument) plus ~2 ulp (v_exp_f32, v_rcp_f32,
// the product): under 1.3e-6 for |g| <= 20, and for g < -20 the value is below 5e-8 * |g|. Special
// values need no guards: g = +inf gives +inf, -inf and NaN give NaN, and very negative g gives -0
// (exp overflows to inf, rcp(inf) = 0), as the reference's quotient does.
__device__ __forceinline__ float silu_lite(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// Two weight codes, one in the low byte of each 16-bit half of p, -> the f16 bit patterns whose
// values are the codes' values / 2^8 (FP8 E4M3: (c & 0x7F) << 7 with the sign moved to bit 15) or
// / 2^14 (FP4 E2M1: (c & 7) << 9, sign to bit 15; the high nibble of each byte is ignored). Exact:
// every E4M3 and E2M1 value, scaled so, is an f16 normal or subnormal.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t fp8_pair_bits(uint32_t p) { return (p + (p & 0x00800080u)) << 7; }
__device__ __forceinline__ uint32_t fp4_pair_bits(uint32_t p) {
    const uint32_t m = p & 0x000F000Fu;
    return (m + 7u * (m & 0x00080008u)) << 9;  // sign bit 3 -> bit 6 before the shift -> bit 15
}

// tanh with the structure of fdlibm's s_tanhf.c (the C library the reference calls through
// std::tanh): expm1-based branches around |x| = 1, saturation at |x| >= 22, identity below 2^-55.
__device__ __forceinline__ float tanh_ref(float x) {
    const float ax = fabsf(x);
    float z;
    if (!(ax < 22.0f)) {
        if (ax != ax) return x + x;
        z = 1.0f;
    } else if (ax < 0x1p-55f) {
        return x;
    } else if (ax >= 1.0f) {
        const float t = expm1f(2.0f * ax);
        z = 1.0f - 2.0f / (t + 2.0f);
    } else {
        const float t = expm1f(-2.0f * ax);
        z = -t / (t + 2.0f);
    }
    return x < 0.0f ? -z : z;
}

// GPT-2 gelu_new (cpu_ops.cpp:20-23), left to right in float.
__device__ __forceinline__ float gelu_ref(float x) {
    const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanh_ref(inner));
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return static_cast<float>(v);
}
// f32 -> f16, one round-to-nearest-even of v as computed (v_cvt_f16_f32). The empty asm keeps the
// backend from folding a multiply that produced v into the conversion as v_fma_mix*_f16(a, b, +0):
// that fused form returns +0 where the product is -0, so x*w = -0 would not round to 0x8000 as the
// reference's separate multiply and conversion do.
__device__ __forceinline__ half_t f16_rne(float v) {
    __asm__("" : "+v"(v));
    return static_cast<half_t>(v);
}

// Conversion to T; for half, f16_rne.
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
    if constexpr (sizeof(T) == 2) return f16_rne(v);
    else return static_cast<T>(v);
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}): a loop with
// compile-time indices, whatever the unroller decides (an element loop over a vector of accumulators
// that is left rolled indexes it at run time and sends the whole array to scratch memory).
template <typename F, int... E>
__device__ __forceinline__ void unrolled_impl(F&& f, std::integer_sequence<int, E...>) {
    (f(std::integral_constant<int, E>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unrolled(F&& f) {
    unrolled_impl(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- DPP cross-lane moves
// dpp_ctrl encodings (GCN3+/CDNA): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_mirror = 0x140, row_half_mirror = 0x141, row_ror:8 = 0x128.
// quad_perm [0,2,0,2] = 0x88 and [1,3,1,3] = 0xDD: lanes 0 / 2 and 1 / 3 of each quad, even lanes of a
// quad taking the first and odd lanes the second.
enum : int {
    kDppQuadXor1 = 0xB1,
    kDppQuadXor2 = 0x4E,
    kDppQuadPairLo = 0x88,
    kDppQuadPairHi = 0xDD,
    kDppRowMirror = 0x140,
    kDppRowHalfMirror = 0x141
};

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b)), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b >> 32)), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

__device__ __forceinline__ double shfl_xor_f64(double v, int mask) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __shfl_xor(static_cast<int>(static_cast<uint32_t>(b)), mask);
    const int hi = __shfl_xor(static_cast<int>(static_cast<uint32_t>(b >> 32)), mask);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Sum over aligned groups of L lanes (L a power of two, 2..64); every lane of a group receives the
// same bits (each step adds a value to its partner's, and IEEE addition is commutative). Must be
// called with all 64 lanes active.
template <int L>
__device__ __forceinline__ double group_sum_f64(double v) {
    static_assert(L >= 2 && L <= 64 && (L & (L - 1)) == 0, "group size");
    v = v + dpp_f64<kDppQuadXor1>(v);
    if constexpr (L >= 4) v = v + dpp_f64<kDppQuadXor2>(v);
    if constexpr (L >= 8) v = v + dpp_f64<kDppRowHalfMirror>(v);
    if constexpr (L >= 16) v = v + dpp_f64<kDppRowMirror>(v);
    if constexpr (L >= 32) v = v + shfl_xor_f64(v, 16);
    if constexpr (L >= 64) v = v + shfl_xor_f64(v, 32);
    return v;
}

// Sum over the whole wavefront, returned wave-uniform: 16-lane DPP all-reduce, then the four row
// sums read back as scalars and added in a fixed order.
__device__ __forceinline__ double wave_sum_f64(double v) {
    v = group_sum_f64<16>(v);
    const double r0 = readlane_f64(v, 0), r1 = readlane_f64(v, 16);
    const double r2 = readlane_f64(v, 32), r3 = readlane_f64(v, 48);
    return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------- workgroup order over the XCDs
// MI355X deals the workgroups of a launch round robin over its 8 XCDs (workgroup b runs on XCD b % 8),
// each with its own L2. For a flat streaming grid, data block xcd_block<R>(b, G) instead of b gives each
// XCD runs of R consecutive data blocks (XCD x: blocks x R .. x R + R - 1 of every group of 8 R), a
// permutation of [0, G); blocks past the last whole group keep their index. R is a power of two, so
// the mapping is shifts and masks. (SwiGLU [8192, 9728], 38,912 workgroups: R = 128 or 256 69.5 us
// against 70.7-70.9 in launch order, R = 16-64 69.9-70.3, 2048 70.7.)
template <int R>
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t G) {
    static_assert(R > 0 && (R & (R - 1)) == 0, "R a power of two");
    const uint32_t full = G / (8u * R) * (8u * R);
    if (b >= full) return b;
    const uint32_t x = b % 8u, k = b / 8u;
    return (k / R) * (8u * R) + x * R + k % R;
}

// ---------------------------------------------------------------- integer division by an invariant
// Granlund & Montgomery (PLDI 1994): q = (umulhi(n, m) + n) >> s with s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1; exact for every 32-bit n.
struct FastDiv {
    uint32_t d, m, s;
};

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
    const uint64_t t = static_cast<uint64_t>(__umulhi(n, f.m)) + n;
    return static_cast<uint32_t>(t >> f.s);
}

}  // namespace neko_hip
