// Device helpers shared by the gfx950 kernels: 16-byte chunk types, f16/f32 conversions, and
// cross-lane reductions built from DPP (no LDS) for 64-wide wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// The reference rounds every float product and sum separately (its portable path has no FMA), so
// kernels must not contract a*b+c into fma. The build passes -ffp-contract=off as well.
#pragma clang fp contract(off)

namespace neko_hip {

constexpr int kWave = 64;

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
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

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return static_cast<float>(v);
}
// Conversion to T; for half this is one round-to-nearest-even (v_cvt_f16_f32 in the default mode).
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
    return static_cast<T>(v);
}

// ---------------------------------------------------------------- DPP cross-lane moves
// dpp_ctrl encodings (GCN3+/CDNA): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_mirror = 0x140, row_half_mirror = 0x141, row_ror:8 = 0x128.
enum : int { kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowMirror = 0x140, kDppRowHalfMirror = 0x141 };

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
