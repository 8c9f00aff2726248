// Qwen3 attention prologue for gfx950: per-head q/k RMSNorm fused with NeoX half-split RoPE, in
// place on the q and k heads of each qkv row (rope.comp:1-55; CPU qwen3_model.cpp:249-253 =
// cpu::rmsNorm per head, cpu_ops.cpp:502-511, then cpu::rope, cpu_ops.cpp:513-524).
//
// Fast path: one wavefront per token row, persistent over tokens. A head of hd elements is spread
// over L lanes; lane l holds the V elements [lV, lV+V) of the first half AND their NeoX partners
// [hd/2 + lV, ...), so the rotation needs no cross-lane exchange. 64/L heads are processed per wave
// pass; all passes of a token are loaded at once, and the next token's heads and cos/sin row are in
// flight while the current token is normalised and rotated. The head's sum of squares (double, like
// the reference) is reduced over its L lanes with DPP only. The norm weights stay in registers for
// all tokens of a wave. V heads are never touched.
//
// Fallback: one 64-thread workgroup per (head, row) staging the head in LDS (any even hd <= 512).
#pragma once

#include <cmath>

#include "internal.h"

namespace neko_hip {

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
    uint16_t* k_cache;  // [>= n_pos][n_kv * hd] f16, or null (no KV store)
    uint16_t* v_cache;
    double inv_hd;  // 1 / hd when hd is a power of two (exact), else 0
};

// V values of type T as f16 at p: bit copies for f16, one RNE rounding each for f32.
template <typename T, int V>
__device__ __forceinline__ void store_f16(uint16_t* p, const typename VecOf<T, V>::V& v) {
    typedef typename VecOf<half_t, V>::V VH;
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<VH*>(p) = __builtin_bit_cast(VH, v);
    } else {
        VH h;
        if constexpr (V == 1) h = static_cast<half_t>(v);
        else
#pragma unroll
            for (int e = 0; e < V; e++) h[e] = static_cast<half_t>(v[e]);
        *reinterpret_cast<VH*>(p) = h;
    }
}

// A lane vector (V elements of T, 2..16 bytes) through a range-checked buffer resource.
template <bool NT, typename VT>
__device__ __forceinline__ VT buf_load16v(BufRes r, uint32_t off) {
    constexpr int aux = NT ? 2 : 0;
    if constexpr (sizeof(VT) == 16) return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, aux));
    else if constexpr (sizeof(VT) == 8) return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, aux));
    else if constexpr (sizeof(VT) == 4) return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, aux));
    else return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, aux));
}
template <bool NT, typename VT>
__device__ __forceinline__ void buf_store16v(BufRes r, uint32_t off, VT v) {
    constexpr int aux = NT ? 2 : 0;
    if constexpr (sizeof(VT) == 16) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uint4v, v), r, off, 0, aux);
    else if constexpr (sizeof(VT) == 8) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(uint2v, v), r, off, 0, aux);
    else if constexpr (sizeof(VT) == 4) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, aux);
    else __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), r, off, 0, aux);
}

// V values of type T as f16 through a buffer resource: bit copies for f16, one RNE rounding each
// for f32.
template <typename T, int V>
__device__ __forceinline__ void store_f16_buf(BufRes r, uint32_t off, const typename VecOf<T, V>::V& v) {
    typedef typename VecOf<half_t, V>::V VH;
    if constexpr (sizeof(T) == 2) {
        buf_store16v<false>(r, off, __builtin_bit_cast(VH, v));
    } else {
        VH h;
        if constexpr (V == 1) h = static_cast<half_t>(v);
        else
#pragma unroll
            for (int e = 0; e < V; e++) h[e] = static_cast<half_t>(v[e]);
        buf_store16v<false>(r, off, h);
    }
}

// The head's norm scale float(1 / sqrt(ss / hd + eps)) (cpu_ops.cpp:508 with C = hd). ss / hd is
// the exact product with 1/hd when hd is a power of two (every Qwen3 head size; the host passes it);
// the reciprocal square root comes from rsqrt_to_float (device.h).
__device__ __forceinline__ float head_scale(const QkArgs& a, double ss) {
    const double m = a.inv_hd != 0.0 ? ss * a.inv_hd : ss / a.hd;
    return rsqrt_to_float(m + static_cast<double>(a.eps));
}

// Head loads non-temporal, stores plain (measured).
template <typename VT>
__device__ __forceinline__ void qk_store(VT* p, VT v) {
    *p = v;
}
template <typename VT>
__device__ __forceinline__ VT qk_load(const VT* p) {
    return load_nt(p);
}

__device__ __forceinline__ bool row_position(const QkArgs& a, int64_t t, int64_t& pos) {
    pos = a.positions ? static_cast<int64_t>(a.positions[t]) : a.pos0 + t;
    return pos >= 0 && pos < a.n_pos;
}

// One token's q/k heads held by one wave: U passes of 64/L heads, each lane V elements of the first
// half of its head and their V partners in the second half.
template <typename T, int V, int U>
struct TokenRegs {
    typedef typename VecOf<T, V>::V VT;
    VT a[U];
    VT b[U];
    float c[V];
    float s[V];
};

template <typename T, int L, int V, int U>
__device__ __forceinline__ void load_token(TokenRegs<T, V, U>& tr, const QkArgs& a, int64_t t, int64_t pos, int p0, int hl,
                                           int hs) {
    typedef typename VecOf<T, V>::V VT;
    constexpr int HPW = kWave / L;
    const int half = a.hd / 2;
    const int i0 = hl * V;
    const float* csr = a.cs + pos * a.hd + 2 * i0;
#pragma unroll
    for (int e = 0; e < V; e++) {
        const float2v c = *reinterpret_cast<const float2v*>(csr + 2 * e);
        tr.c[e] = c[0];
        tr.s[e] = c[1];
    }
    const T* row = static_cast<const T*>(a.qkv) + t * a.stride;
    const int nh = a.n_q + a.n_kv;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int head = p0 + u * HPW + hs;
        tr.a[u] = VT{};
        tr.b[u] = VT{};
        if (head < nh) {
            const T* hp = row + static_cast<int64_t>(head) * a.hd + i0;
            tr.a[u] = qk_load(reinterpret_cast<const VT*>(hp));
            tr.b[u] = qk_load(reinterpret_cast<const VT*>(hp + half));
        }
    }
}

template <typename T, int L, int V, int U>
__device__ __forceinline__ void rotate_token(const TokenRegs<T, V, U>& tr, const QkArgs& a, int64_t t, int p0, int hl,
                                             int hs, bool norm, const float (&wqa)[V], const float (&wqb)[V],
                                             const float (&wka)[V], const float (&wkb)[V]) {
    typedef typename VecOf<T, V>::V VT;
    constexpr int HPW = kWave / L;
    const int half = a.hd / 2;
    const int i0 = hl * V;
    const int nh = a.n_q + a.n_kv;
    T* row = static_cast<T*>(a.qkv) + t * a.stride;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int head = p0 + u * HPW + hs;
        float fa[V], fb[V];
#pragma unroll
        for (int e = 0; e < V; e++) {
            if constexpr (V == 1) {
                fa[e] = to_f32(tr.a[u]);
                fb[e] = to_f32(tr.b[u]);
            } else {
                fa[e] = to_f32(tr.a[u][e]);
                fb[e] = to_f32(tr.b[u][e]);
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
            const float r = head_scale(a, ss);
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
            const float x0 = fa[e] * tr.c[e] - fb[e] * tr.s[e];
            const float x1 = fa[e] * tr.s[e] + fb[e] * tr.c[e];
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
            qk_store(reinterpret_cast<VT*>(hp), oa);
            qk_store(reinterpret_cast<VT*>(hp + half), ob);
        }
    }
}

// Rolling pipeline for tokens whose heads fit in U passes: a wave holds one token's q/k heads in
// registers; as each pass of token t is normalised, rotated and stored, the same registers receive
// that pass of the wave's next token. A whole token of loads is therefore always in flight behind
// the token being computed, with one token's worth of data registers, and because every load is
// issued after the stores it follows, waiting for it never waits on later stores.
// Wave w takes tokens w, w + nw, ... (nw waves in the grid; at most 64 each, which the host
// guarantees). With S > 1 a token is S work items of U passes each (item i: token i / S, passes
// (i % S) * U ...), and wave w takes items w, w + nw, ... -- all of one part, as nw is a multiple of
// S (the host's grid): the fused KV store at six or eight passes runs as two items of three or four,
// which halves a wave's data registers and serial passes (8192 tokens of 32 + 8 + 8 heads x 128:
// 5 waves per SIMD instead of 3, 38.0-39.2 us against 39.2-39.4 on the same buffers, bit-identical),
// and a token of 10-16 passes (an even count) as two items of half of them, which the one-token roll
// cannot hold (f32 rows of 32 + 8 heads x 128, ten passes: 51.5 us against 59.2 on the batch kernel).
// Wave w's first item is taken from workgroup xcd_block<64>(w / 4) rather than w / 4, so that the
// workgroups of each XCD take runs of consecutive rows.
// Everything a token needs besides its row is fetched ahead of it: the positions of all
// of the wave's tokens in one vector load at the start (lane k holds token k's), and the cos/sin row
// of the next token, loaded with one coalesced load spread over the lanes (8 bytes each at hd 128)
// and staged in the wave's own LDS double buffer, from which every pass reads its (c, s) pairs. The
// norm weights are staged once per wave in its own LDS copy, so no wave waits on a barrier before its
// first row loads go out. Row data moves through range-checked buffer resources (device.h): lanes past
// the last head load zeros and their stores are dropped, so no load or store is under a per-lane
// branch, and the first and the last token of a wave are peeled, so the loop issues every load
// unconditionally -- together these keep the compiler's memory-counter waits at "this pass's data"
// rather than "everything outstanding". A token whose position lies outside the table is written
// back unchanged (and not stored to the caches).
// Waves per SIMD: 4 where the token's data registers leave room -- at most 40 of them (32 with the KV
// store, whose cache addressing needs more), found to compile without spills -- else 3.
template <typename T, int V, int U, bool KV>
constexpr int qk_waves() {
    return 2 * U * V * static_cast<int>(sizeof(T)) <= (KV ? 128 : 160) ? 4 : 3;
}

// Tokens one wave of qk_rope_roll_kernel may take (one position per lane).
constexpr int kQkMaxTokensPerWave = 64;

// What the kernel's scalar load of its first position reads when the call has no positions array.
static __device__ const int32_t kQkNoPosition = 0;

template <typename T, int L, int V, int U, bool KV, int S = 1>
__global__ __launch_bounds__(256, (qk_waves<T, V, U, KV>())) void qk_rope_roll_kernel(QkArgs a) {
    constexpr int HPW = kWave / L;  // heads per wave pass
    constexpr int HD = 2 * L * V;   // the head size (a power of two): offsets and 1/HD are constants
    constexpr int PL = (L * V + 63) / 64;  // (cos, sin) pairs each lane stages per row
    constexpr int WQ = 2 * HD > 256 ? 2 * HD : 256;  // floats of a wave's weight copy (64 lanes x 4 at least)
    typedef typename VecOf<T, V>::V VT;
    __shared__ __align__(16) float wsh[4][WQ];
    __shared__ __align__(16) float csl[4][2][HD];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, kept in SGPRs
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    // First work item (token, part): workgroups in runs of 64 per XCD (xcd_block; 1.3% faster than
    // launch order at the Qwen3-4B prefill shape, measured twice).
    const int64_t item0 = static_cast<int64_t>(xcd_block<64>(blockIdx.x, gridDim.x)) * 4 + wave;
    const int64_t items = S == 1 ? a.rows : a.rows * S;
    if (item0 >= items) return;  // wave-uniform
    const int ntok = static_cast<int>((items - 1 - item0) / nw) + 1;
    const int part = S == 1 ? 0 : static_cast<int>(item0 % S);  // the same for all of a wave's items (nw % S == 0)
    const int64_t t0 = S == 1 ? item0 : item0 / S;  // its first token; the next ones follow tnw apart
    const int64_t tnw = S == 1 ? nw : nw / S;
    const int hl = lane % L;
    const int hs = lane / L;
    constexpr int half = HD / 2;
    const int i0 = hl * V;
    const int nqk = a.n_q + a.n_kv;
    const int nh = KV ? nqk + a.n_kv : nqk;  // with the KV store, the v heads ride along as extra passes
    const int64_t kvw = static_cast<int64_t>(a.n_kv) * HD;
    // Byte extents: the heads a wave loads (v included with the KV store) and the ones it writes back.
    const int hb = part * U * HPW;  // this part's first head
    const int hl_end = S == 1 || nh < hb + U * HPW ? nh : hb + U * HPW;
    const int hs_end = S == 1 || nqk < hb + U * HPW ? nqk : hb + U * HPW;
    const uint32_t load_bytes = static_cast<uint32_t>(hl_end > hb ? hl_end - hb : 0) * HD * sizeof(T);
    const uint32_t store_bytes = static_cast<uint32_t>(hs_end > hb ? hs_end - hb : 0) * HD * sizeof(T);
    const uint32_t cache_bytes = static_cast<uint32_t>(kvw) * 2u;
    const bool norm = a.wqk != nullptr;
    float* const cb = &csl[wave][0][0];
    const float* const wl = &wsh[wave][0];
    auto row_of = [&](int64_t t) __attribute__((always_inline)) -> const T* {
        return static_cast<const T*>(a.qkv) + t * a.stride + static_cast<int64_t>(hb) * HD;
    };
    // Byte offsets of this lane's vector of pass u in a row (first half; the partner is half later).
    auto off = [&](int u) __attribute__((always_inline)) -> uint32_t {
        return static_cast<uint32_t>((u * HPW + hs) * HD + i0) * sizeof(T);
    };

    // Issued first: the wave's positions (lane k: token k's), its weight copy, then the first token's
    // row -- none of them waits for another.
    int32_t posv = 0;
    if (a.positions) posv = a.positions[t0 + static_cast<int64_t>(lane < ntok ? lane : ntok - 1) * tnw];
    // The first token's position once more, through the scalar cache (a uniform address in the constant
    // address space: s_load, issued here and waited for only after the row loads below): the first
    // cos/sin row waits on it, and a scalar load returns well before the vector load above.
    const int32_t* const pfirst = a.positions ? a.positions + t0 : &kQkNoPosition;
    const int32_t pos32 = ((const __attribute__((address_space(4))) int32_t*)pfirst)[0];  // (a C cast: address spaces)
    float4v wv{};
    if (norm) wv = buf_load16<false, float4v>(buf_res(a.wqk, 2 * HD * 4u), lane * 16u);
    VT A[U], B[U];
    auto load_pass = [&](const BufRes& r, int u) __attribute__((always_inline)) {
        A[u] = buf_load16v<true, VT>(r, off(u));
        B[u] = buf_load16v<true, VT>(r, off(u) + half * sizeof(T));
    };
    // Token k's position (wave-uniform) and whether it indexes the table.
    auto pos_of = [&](int k) __attribute__((always_inline)) -> int64_t {
        return a.positions ? static_cast<int64_t>(__builtin_amdgcn_readlane(posv, k)) : a.pos0 + t0 + k * tnw;
    };
    auto in_table = [&](int64_t p) __attribute__((always_inline)) -> bool { return p >= 0 && p < a.n_pos; };
    // Pairs lane, lane + 64, ... of the row at `pos` (row 0 for a position outside the table): loaded
    // into r, then stored to buffer b.
    auto cs_load = [&](int64_t pos, float2v (&r)[PL]) __attribute__((always_inline)) {
        const float* row = a.cs + (in_table(pos) ? pos : 0) * HD;
#pragma unroll
        for (int k = 0; k < PL; k++) {
            const int p = lane + 64 * k;
            if (p < L * V) r[k] = *reinterpret_cast<const float2v*>(row + 2 * p);
        }
    };
    auto cs_store = [&](int b, const float2v (&r)[PL]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < PL; k++) {
            const int p = lane + 64 * k;
            if (p < L * V) *reinterpret_cast<float2v*>(cb + b * HD + 2 * p) = r[k];
        }
    };

    // Normalises, rotates and stores every pass of token k (cos/sin from LDS buffer `buf`); with
    // `more`, refills each pass's registers with token k + 1's right after its stores.
    auto step = [&](int k, int buf, bool more) __attribute__((always_inline)) {
        const int64_t t = t0 + k * tnw;
        const int64_t pos = pos_of(k);
        const bool valid = in_table(pos);
        const float* cr = cb + buf * HD + 2 * i0;  // this lane's V (cos, sin) pairs
        const BufRes st = buf_res(row_of(t), store_bytes);
        const BufRes ld = buf_res(row_of(more ? t + tnw : t), load_bytes);
        // The cache rows of this token's position (only written with the KV store, and only for a
        // position inside the table: otherwise the resources are empty and every store drops).
        const int64_t cpos = valid ? pos : 0;
        const uint32_t cbytes = valid ? cache_bytes : 0u;
        const BufRes kc = buf_res(KV ? static_cast<const void*>(a.k_cache + cpos * kvw) : a.qkv, cbytes);
        const BufRes vc = buf_res(KV ? static_cast<const void*>(a.v_cache + cpos * kvw) : a.qkv, cbytes);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int head = hb + u * HPW + hs;  // absolute head index
            VT oa = A[u], ob = B[u];
            if (valid) {
                float fa[V], fb[V];
#pragma unroll
                for (int e = 0; e < V; e++) {
                    if constexpr (V == 1) {
                        fa[e] = to_f32(A[u]);
                        fb[e] = to_f32(B[u]);
                    } else {
                        fa[e] = to_f32(A[u][e]);
                        fb[e] = to_f32(B[u][e]);
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
                    const float r = rsqrt_to_float(ss * (1.0 / HD) + static_cast<double>(a.eps));
                    const float* w = wl + (head < a.n_q ? 0 : HD) + i0;
#pragma unroll
                    for (int e = 0; e < V; e++) {
                        fa[e] = fa[e] * r * w[e];
                        fb[e] = fb[e] * r * w[half + e];
                    }
                }
#pragma unroll
                for (int e = 0; e < V; e++) {
                    float c, s;
                    if constexpr (V == 1) {
                        const float2v v = *reinterpret_cast<const float2v*>(cr);
                        c = v[0];
                        s = v[1];
                    } else {
                        const float4v v = *reinterpret_cast<const float4v*>(cr + 2 * (e & ~1));
                        c = v[2 * (e & 1)];
                        s = v[2 * (e & 1) + 1];
                    }
                    const float x0 = fa[e] * c - fb[e] * s;
                    const float x1 = fa[e] * s + fb[e] * c;
                    if constexpr (V == 1) {
                        oa = from_f32<T>(x0);
                        ob = from_f32<T>(x1);
                    } else {
                        oa[e] = from_f32<T>(x0);
                        ob[e] = from_f32<T>(x1);
                    }
                }
            }
            // q and k heads back in place (v heads and lanes past the last head fall outside `st`).
            buf_store16v<false>(st, off(u), oa);
            buf_store16v<false>(st, off(u) + half * sizeof(T), ob);
            if constexpr (KV) {
                // Rotated k heads to the k cache row, untouched v heads to the v cache row; each
                // resource's range drops the other heads' stores (their offsets wrap past it).
                const uint32_t ko = static_cast<uint32_t>((head - a.n_q) * HD + i0) * 2u;
                const uint32_t vo = static_cast<uint32_t>((head - nqk) * HD + i0) * 2u;
                store_f16_buf<T, V>(kc, ko, oa);
                store_f16_buf<T, V>(kc, ko + half * 2u, ob);
                store_f16_buf<T, V>(vc, vo, A[u]);
                store_f16_buf<T, V>(vc, vo + half * 2u, B[u]);
            }
            if (more) load_pass(ld, u);
        }
    };

    // The first token's row data goes out first, then the weight copy and that token's cos/sin row
    // (loading the cos/sin row first waits for the position before any row load is issued: measured
    // 0.8 us slower at the Qwen3-4B prefill shape), whose position comes from the scalar load above.
    {
        float2v r[PL];
        const BufRes ld = buf_res(row_of(t0), load_bytes);
#pragma unroll
        for (int u = 0; u < U; u++) load_pass(ld, u);
        __builtin_amdgcn_sched_barrier(0);  // every row load issued before the wait for the position
        const int64_t pos_first = a.positions ? static_cast<int64_t>(pos32) : a.pos0 + t0;
        if (norm) {
            *reinterpret_cast<float4v*>(&wsh[wave][lane * 4]) = wv;
            for (int i = 256 + lane * 4; i < 2 * HD; i += 256)
                *reinterpret_cast<float4v*>(&wsh[wave][i]) = *reinterpret_cast<const float4v*>(a.wqk + i);
        }
        cs_load(pos_first, r);
        cs_store(0, r);
    }
    // Token k with a next token: its passes, the refills, and the next cos/sin row staged in the other
    // LDS buffer (this wave's own LDS operations run in order, so the next step's reads see it).
    int k = 0;
    auto advance = [&]() __attribute__((always_inline)) {
        float2v ncs[PL];
        cs_load(pos_of(k + 1), ncs);
        step(k, k & 1, true);
        cs_store((k & 1) ^ 1, ncs);
        k++;
    };
    // The first step is peeled so that the loop is entered with the memory ops of a step outstanding,
    // as after each iteration (the compiler's waits then hold for both ways into the loop).
    if (k + 1 < ntok) {
        advance();
        while (k + 1 < ntok) advance();
    }
    step(k, k & 1, false);
}

// Tokens with more heads than U passes: persistent waves, each token in batches of U passes, the norm
// weights in registers.
template <typename T, int L, int V, int U>
__global__ __launch_bounds__(256) void qk_rope_batch_kernel(QkArgs a) {
    constexpr int HPW = kWave / L;  // heads per wave pass
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    const int hl = lane % L;
    const int hs = lane / L;
    const int half = a.hd / 2;
    const int i0 = hl * V;
    const bool norm = a.wqk != nullptr;
    float wqa[V], wqb[V], wka[V], wkb[V];
#pragma unroll
    for (int e = 0; e < V; e++) {
        wqa[e] = norm ? a.wqk[i0 + e] : 1.0f;
        wqb[e] = norm ? a.wqk[half + i0 + e] : 1.0f;
        wka[e] = norm ? a.wqk[a.hd + i0 + e] : 1.0f;
        wkb[e] = norm ? a.wqk[a.hd + half + i0 + e] : 1.0f;
    }
    const int nh = a.n_q + a.n_kv;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave; t < a.rows; t += nw) {
        int64_t pos;
        if (!row_position(a, t, pos)) continue;  // rows outside the table stay untouched
        for (int p0 = 0; p0 < nh; p0 += HPW * U) {
            TokenRegs<T, V, U> cur;
            load_token<T, L, V, U>(cur, a, t, pos, p0, hl, hs);
            rotate_token<T, L, V, U>(cur, a, t, p0, hl, hs, norm, wqa, wqb, wka, wkb);
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

// The rolling kernel when a token's heads fit in U <= 8 passes, else (without the KV store) the
// batch kernel; with the KV store there is no batch form and the caller runs the unfused pair.
template <typename T, int L, int V, int U, bool KV>
QkKernel pick_fit(bool fit) {
    if constexpr (KV) return fit ? qk_rope_roll_kernel<T, L, V, U, true> : nullptr;
    else return fit ? qk_rope_roll_kernel<T, L, V, U, false> : qk_rope_batch_kernel<T, L, V, U>;
}

// *split = the work items per token: 2 for the fused KV store at six or eight passes, and for 16-byte
// lane vectors at an even pass count from 10 to 16 (f32 rows of 32 + 8 heads x 128: ten passes, two
// rolling items of five instead of the batch kernel); else 1.
template <typename T, int L, int V, bool KV>
QkKernel pick_u(int passes, int* split) {
    *split = 1;
    if constexpr (KV) {
        if (passes == 6 || passes == 8) {
            *split = 2;
            return passes == 6 ? qk_rope_roll_kernel<T, L, V, 3, true, 2> : qk_rope_roll_kernel<T, L, V, 4, true, 2>;
        }
    }
    if constexpr (V == Chunk16<T>::N) {
        if (passes >= 10 && passes <= 16 && passes % 2 == 0) {
            *split = 2;
            switch (passes / 2) {
                case 5: return qk_rope_roll_kernel<T, L, V, 5, KV, 2>;
                case 6: return qk_rope_roll_kernel<T, L, V, 6, KV, 2>;
                case 7: return qk_rope_roll_kernel<T, L, V, 7, KV, 2>;
                case 8: return qk_rope_roll_kernel<T, L, V, 8, KV, 2>;
            }
        }
    }
    switch (passes) {
        case 1: return pick_fit<T, L, V, 1, KV>(true);
        case 2: return pick_fit<T, L, V, 2, KV>(true);
        case 3: return pick_fit<T, L, V, 3, KV>(true);
        case 4: return pick_fit<T, L, V, 4, KV>(true);
        case 5: return pick_fit<T, L, V, 5, KV>(true);
        case 6: return pick_fit<T, L, V, 6, KV>(true);
        case 7: return pick_fit<T, L, V, 7, KV>(true);
        case 8: return pick_fit<T, L, V, 8, KV>(true);
    }
    return pick_fit<T, L, V, 8, KV>(false);
}

template <typename T, int V, bool KV>
QkKernel pick_l(int L, int nh, int* split) {
    const int passes = (nh + kWave / L - 1) / (kWave / L);
    switch (L) {
        case 2: return pick_u<T, 2, V, KV>(passes, split);
        case 4: return pick_u<T, 4, V, KV>(passes, split);
        case 8: return pick_u<T, 8, V, KV>(passes, split);
        case 16: return pick_u<T, 16, V, KV>(passes, split);
        case 32: return pick_u<T, 32, V, KV>(passes, split);
        case 64:
            if constexpr (2 * 64 * V <= 512) return pick_u<T, 64, V, KV>(passes, split);  // head sizes up to 512
            return nullptr;
    }
    return nullptr;
}

template <typename T, bool KV>
QkKernel pick_lv(int L, int V, int nh, int* split) {
    *split = 1;
    // The fused KV store exists for 16-byte lane vectors only (every power-of-two head size); other
    // shapes take the unfused pair.
    if constexpr (KV) {
        return V == Chunk16<T>::N ? pick_l<T, Chunk16<T>::N, true>(L, nh, split) : nullptr;
    } else {
        // Lane vectors are at most 16 bytes (the launcher's limit): 8 halves or 4 floats.
        switch (V) {
            case 1: return pick_l<T, 1, false>(L, nh, split);
            case 2: return pick_l<T, 2, false>(L, nh, split);
            case 4: return pick_l<T, 4, false>(L, nh, split);
            case 8:
                if constexpr (sizeof(T) == 2) return pick_l<T, 8, false>(L, nh, split);
                return nullptr;
        }
        return nullptr;
    }
}

// Kernel pickers per activation type (qk_rope_f16.hip, qk_rope_f32.hip): the kernel for a head
// split into L lanes of V elements and nh heads per row, with or without the fused KV store, and in
// *split the work items it makes of each token (the roll kernel's S).
QkKernel pick_qk_f16(int L, int V, int nh, bool kv, int* split);
QkKernel pick_qk_f32(int L, int V, int nh, bool kv, int* split);

}  // namespace neko_hip
