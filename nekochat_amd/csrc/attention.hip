// Causal grouped-query attention over f16 KV caches for gfx950 (cpu::attention, cpu_ops.cpp:544-575;
// the GPU kernel Attention, attention.comp, dispatched by qwen3_model.cpp:317 and gpt2_model.cpp:255):
// for token t at position pos0 + t and query head h, out = sum_j softmax_j(scale * q_h . k_j) v_j over
// cache rows j <= pos0 + t, k_j / v_j being kv head h / (n_head / n_kv) of those rows.
//
// A workgroup of four waves per work item (token, kv head, block of up to four of the query heads that
// share it, split of the keys), the item's steps of keys dealt round robin to its waves. Lane = (key
// residue, 16-byte chunk of the head): each load instruction reads whole K or V head rows (16 lanes per
// 256-byte row of a 128-dimension head), and each lane keeps its chunk of the item's q rows in
// registers. A step issues all of its K and V loads first; the scores are the lanes' 8-dimension
// partial dots summed over a row's lanes by DPP; the softmax is the streaming form (running maximum;
// the sum and the accumulators rescaled when it grows), lane = key, its weights passed through LDS;
// then each lane adds its keys' weighted v chunks. The heads of a block share every K and V load. At
// the end each wave sums its accumulators over the key residues and the waves merge through LDS.
// When tokens x kv heads x head blocks give too few waves to fill the chip (decode: one token), each
// token's keys split over several items that write (maximum, sum, accumulators) to the context's
// workspace, and attn_merge_kernel combines them. The reference's CPU loop and its shader already sum
// in different orders; any order here is one more within the same bound.
#include <algorithm>
#include <cmath>

#include "internal.h"

namespace neko_hip {
namespace {

constexpr int kAttnHeads = 4;              // query heads per work item, at most (HB = 4 or 1)
constexpr int kAttnWaves = 4;              // waves per work item (its steps interleaved)
constexpr int64_t kAttnTargetWaves = 4096;  // keys split until a launch holds about this many waves
constexpr int64_t kAttnMaxSplits = 1024;    // the merge kernel's LDS weights
constexpr int64_t kAttnOneHeadBytes = int64_t{32} << 20;  // K + V bytes up to which items take one head

struct AttnArgs {
    const void* q;
    int64_t qs;  // q row stride (elements)
    const uint16_t* kc;
    const uint16_t* vc;
    int64_t kvw;  // cache row width (halves) = n_kv * hd
    void* out;
    int64_t os;  // out row stride (elements)
    int64_t T;
    int64_t pos0;
    int n_head;
    int n_kv;
    int group;    // n_head / n_kv
    int hblocks;  // ceil(group / HB): the head blocks per kv head
    int hd;
    float scale;
    int splits;          // key splits per (token, kv head, head block)
    int64_t split_keys;  // keys per split, a multiple of the kernel's step
    float* part;         // splits > 1: [T][n_head][splits][hd + 2] = (max, sum, accumulators)
};

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Maximum / sum over the wave, returned wave-uniform (16-lane DPP all-reduce, then the four row results
// combined in a fixed order). All 64 lanes active.
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
    return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v = v + dpp_f32<kDppQuadXor1>(v);
    v = v + dpp_f32<kDppQuadXor2>(v);
    v = v + dpp_f32<kDppRowHalfMirror>(v);
    v = v + dpp_f32<kDppRowMirror>(v);
    return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

// Eight halves of a cache row at p -- dimensions d .. d + 7 of a head, those at or past hd read as 0 --
// packed two to a register. AL: hd % 8 == 0 and the cache 16-byte aligned, so one 16-byte load.
template <bool AL>
__device__ __forceinline__ void load8(const uint16_t* p, int d, int hd, uint32_t (&r)[4]) {
    if constexpr (AL) {
        const uint4v v = d < hd ? *reinterpret_cast<const uint4v*>(p + d) : uint4v{0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = v[e];
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t lo = d + 2 * e < hd ? p[d + 2 * e] : 0u;
            const uint32_t hi = d + 2 * e + 1 < hd ? p[d + 2 * e + 1] : 0u;
            r[e] = lo | (hi << 16);
        }
    }
}

__device__ __forceinline__ float half_at(const uint32_t (&r)[4], int e) {
    const half2v h = __builtin_bit_cast(half2v, r[e >> 1]);
    return static_cast<float>(h[e & 1]);
}

// Sum over aligned groups of DC lanes (DC = 8, 16 or 32), every lane of a group receiving the sum.
template <int DC>
__device__ __forceinline__ float group_sum_f32(float v) {
    v = v + dpp_f32<kDppQuadXor1>(v);
    v = v + dpp_f32<kDppQuadXor2>(v);
    v = v + dpp_f32<kDppRowHalfMirror>(v);
    if constexpr (DC >= 16) v = v + dpp_f32<kDppRowMirror>(v);
    if constexpr (DC >= 32) v = v + __shfl_xor(v, 16);
    return v;
}

// Partial results of a key split (splits > 1): the accumulators [T][n_head][splits][hd] at part, then
// (max, sum) pairs [T][n_head][splits][2] after them.
__device__ __forceinline__ float* part_acc(const AttnArgs& a, int64_t th, int split) {
    return a.part + (th * a.splits + split) * a.hd;
}
__device__ __forceinline__ float* part_ml(const AttnArgs& a, int64_t th, int split) {
    return a.part + a.T * a.n_head * a.splits * a.hd + (th * a.splits + split) * 2;
}

// Lane layout: lane = (key residue r, chunk c) -- 16-byte chunk c (dimensions 8c .. 8c + 7) of key
// rows j0 + KR u + r, u = 0 .. KU - 1 -- so each load instruction reads KR whole head rows of K or V
// (16 lanes per 256-byte row of a 128-dimension head) and each lane keeps its chunk of the q rows in
// registers. HDP: the head size rounded up to 64, 128 or 256 (DC = HDP / 8 chunks); a step is KR x 8
// keys (64 / 32 / 16): eight K and eight V loads per lane, issued before the previous step's
// arithmetic. NW waves per workgroup share one work item, its steps
// dealt round robin; their states merge through LDS at the end.
template <typename TQ, int HDP, bool AL, int NW, int HB, bool PF>
__global__ __launch_bounds__(64 * NW) void attn_kernel(AttnArgs a) {
    constexpr int DC = HDP / 8;
    constexpr int KR = 64 / DC;
    constexpr int KU = 8;
    constexpr int STEP = KR * KU;
    __shared__ float ssh[NW][HB][STEP];  // the step's scores by key, then its weights by (r, u)
    __shared__ float msh[NW][HB], lsh[NW][HB];
    __shared__ __align__(16) float ash[NW][HB][HDP];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int c = lane % DC, r = lane / DC;
    // Item index -> (token, kv head, head block, split), in 32 bits (the host keeps items below 2^31;
    // 64-bit division is a loop on this target). The latest tokens (the most keys) first.
    const uint32_t per_t = static_cast<uint32_t>(a.n_kv) * static_cast<uint32_t>(a.hblocks) * static_cast<uint32_t>(a.splits);
    const uint32_t item = blockIdx.x;
    const uint32_t tr = item / per_t;
    const int64_t t = a.T - 1 - tr;
    uint32_t rest = item - tr * per_t;
    const int split = static_cast<int>(rest % static_cast<uint32_t>(a.splits));
    rest /= static_cast<uint32_t>(a.splits);
    const int hb = static_cast<int>(rest % static_cast<uint32_t>(a.hblocks));
    const int g = static_cast<int>(rest / static_cast<uint32_t>(a.hblocks));
    const int h0 = g * a.group + hb * HB;
    const int nh = min(HB, a.group - hb * HB);
    const int hd = a.hd;
    const int64_t L = a.pos0 + t + 1;
    const int64_t k0 = static_cast<int64_t>(split) * a.split_keys;
    const int64_t k1 = min(L, k0 + a.split_keys);

    // This lane's chunk of each q row, f32.
    const TQ* qrow = static_cast<const TQ*>(a.q) + t * a.qs + static_cast<int64_t>(h0) * hd;
    float qv[HB][8];
#pragma unroll
    for (int i = 0; i < HB; i++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = 8 * c + e;
            qv[i][e] = i < nh && d < hd ? to_f32(qrow[static_cast<int64_t>(i) * hd + d]) : 0.0f;
        }
    float m[HB], l[HB], acc[HB][8];
#pragma unroll
    for (int i = 0; i < HB; i++) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[i][e] = 0.0f;
    }
    const uint16_t* kbase = a.kc + static_cast<int64_t>(g) * hd;
    const uint16_t* vbase = a.vc + static_cast<int64_t>(g) * hd;
    float(*sw)[STEP] = ssh[wave];

    // The K and V rows of the step at j0 (rows j0 + KR u + r; past k1: row k1 - 1, not counted). Nothing
    // here uses the loaded registers, so the loads stay in flight.
    auto load_step = [&](int64_t j0, uint32_t(&kr)[KU][4], uint32_t(&vr)[KU][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < KU; u++) load8<AL>(kbase + min(j0 + KR * u + r, k1 - 1) * a.kvw, 8 * c, hd, kr[u]);
#pragma unroll
        for (int u = 0; u < KU; u++) load8<AL>(vbase + min(j0 + KR * u + r, k1 - 1) * a.kvw, 8 * c, hd, vr[u]);
    };
    auto step = [&](int64_t j0, const uint32_t(&kr)[KU][4], const uint32_t(&vr)[KU][4]) __attribute__((always_inline)) {
        // Scores: each lane's 8-dimension partial dot, summed over the DC lanes of its key row.
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int key = KR * u + r;
            const bool valid = j0 + key < k1;
#pragma unroll
            for (int i = 0; i < HB; i++) {
                if (i >= nh) break;
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) p = __builtin_fmaf(qv[i][e], half_at(kr[u], e), p);
                p = group_sum_f32<DC>(p);
                sw[i][key] = valid ? p * a.scale : -INFINITY;  // the DC lanes of the key store the same bits
            }
        }
        wave_sync_lds();
        // Streaming softmax per head, lane = key; the weights go back to LDS by (r, u).
#pragma unroll
        for (int i = 0; i < HB; i++) {
            if (i >= nh) break;
            const float s = lane < STEP ? sw[i][lane] : -INFINITY;
            const float mn = fmaxf(m[i], wave_max_f32(s));  // finite: the step holds a valid key
            const float corr = expf(m[i] - mn);             // 0 on the wave's first step (m = -inf)
            const float p = expf(s - mn);                   // 0 for keys past k1
            l[i] = l[i] * corr + wave_sum_f32(p);
#pragma unroll
            for (int e = 0; e < 8; e++) acc[i][e] *= corr;
            m[i] = mn;
            wave_sync_lds();  // every lane has read its score before the weights overwrite them
            if (lane < STEP) sw[i][(lane % KR) * KU + lane / KR] = p;
        }
        wave_sync_lds();
        // Weighted v rows: this lane's keys KR u + r, chunk c (a key past k1 adds nothing: its row is
        // another key's, and 0 x inf would be NaN).
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const bool valid = j0 + KR * u + r < k1;
            float vf[8];
#pragma unroll
            for (int e = 0; e < 8; e++) vf[e] = valid ? half_at(vr[u], e) : 0.0f;
#pragma unroll
            for (int i = 0; i < HB; i++) {
                if (i >= nh) break;
                const float w = sw[i][r * KU + u];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[i][e] = __builtin_fmaf(w, vf[e], acc[i][e]);
            }
        }
        wave_sync_lds();  // the next step rewrites sw
    };
    // Steps j0, j0 + NW STEP, ...; with PF (waves of several steps) the next step's loads are issued
    // before each step's arithmetic, in two register sets that alternate (no copy of registers a load
    // is still filling; the last prefetch re-reads row k1 - 1). Without PF each step loads, then
    // computes, in half the registers.
    const int64_t stride = static_cast<int64_t>(NW) * STEP;
    int64_t j0 = k0 + static_cast<int64_t>(wave) * STEP;
    if constexpr (!PF) {
        for (; j0 < k1; j0 += stride) {
            uint32_t ka[KU][4], va[KU][4];
            load_step(j0, ka, va);
            step(j0, ka, va);
        }
    } else if (j0 < k1) {
        uint32_t ka[KU][4], va[KU][4], kb[KU][4], vb[KU][4];
        load_step(j0, ka, va);
        for (;;) {
            load_step(j0 + stride, kb, vb);
            step(j0, ka, va);
            j0 += stride;
            if (j0 >= k1) break;
            load_step(j0 + stride, ka, va);
            step(j0, kb, vb);
            j0 += stride;
            if (j0 >= k1) break;
        }
    }

    // The wave's accumulators: summed over its KR key residues (lanes DC apart), then through LDS the
    // waves merge -- wave i merging head i, in wave order.
#pragma unroll
    for (int i = 0; i < HB; i++) {
        if (i >= nh) break;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[i][e];
#pragma unroll
            for (int x = DC; x < 64; x *= 2) v += __shfl_xor(v, x);
            acc[i][e] = v;
        }
        if (r == 0) {
#pragma unroll
            for (int e = 0; e < 8; e++) ash[wave][i][8 * c + e] = acc[i][e];
        }
        if (lane == 0) {
            msh[wave][i] = m[i];
            lsh[wave][i] = l[i];
        }
    }
    __syncthreads();
    constexpr int DPL = HDP / 64;
    const int d0 = lane * DPL;
    for (int i = wave; i < nh; i += NW) {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) mx = fmaxf(mx, msh[w][i]);
        float sum = 0.0f, o[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) o[e] = 0.0f;
        if (mx != -INFINITY) {  // an empty split (k0 >= L) keeps max -inf, sum 0
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float ww = expf(msh[w][i] - mx);  // a wave without steps: 0
                sum = __builtin_fmaf(ww, lsh[w][i], sum);
#pragma unroll
                for (int e = 0; e < DPL; e++) o[e] = __builtin_fmaf(ww, ash[w][i][d0 + e], o[e]);
            }
        }
        const int64_t th = t * a.n_head + h0 + i;
        if (a.splits == 1) {
            TQ* orow = static_cast<TQ*>(a.out) + t * a.os + static_cast<int64_t>(h0 + i) * hd;
            const float inv = 1.0f / sum;
#pragma unroll
            for (int e = 0; e < DPL; e++)
                if (d0 + e < hd) orow[d0 + e] = from_f32<TQ>(o[e] * inv);
        } else {
            float* pa = part_acc(a, th, split);
#pragma unroll
            for (int e = 0; e < DPL; e++)
                if (d0 + e < hd) pa[d0 + e] = o[e];
            if (lane == 0) {
                float* pm = part_ml(a, th, split);
                pm[0] = mx;
                pm[1] = sum;
            }
        }
    }
}

// Merges the key splits of one (token, head) per workgroup of 256 threads: M = the largest split
// maximum, each split weighted by exp(max - M); the sums and the accumulators added over the splits
// (threads over splits and dimensions, then the waves and groups in a fixed order); out = acc / sum.
template <typename TQ>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    constexpr int kPer = kAttnMaxSplits / 256;  // splits per thread, at most
    __shared__ float wsh[kAttnMaxSplits];
    __shared__ float red[2][4];
    __shared__ float osh[8][256];
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6;
    const int64_t th = blockIdx.x;
    const uint32_t tq = blockIdx.x / static_cast<uint32_t>(a.n_head);  // 32-bit: T * n_head < 2^31
    const int64_t t = tq;
    const int h = static_cast<int>(blockIdx.x - tq * static_cast<uint32_t>(a.n_head));
    const int hd = a.hd, S = a.splits;
    float ms[kPer], ls[kPer];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const int s = tid + 256 * k;
        const float* pm = part_ml(a, th, min(s, S - 1));
        ms[k] = s < S ? pm[0] : -INFINITY;
        ls[k] = s < S ? pm[1] : 0.0f;
        mx = fmaxf(mx, ms[k]);
    }
    mx = wave_max_f32(mx);
    if ((tid & 63) == 0) red[0][wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));  // finite: split 0 holds key 0
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const int s = tid + 256 * k;
        const float ws = expf(ms[k] - mx);  // an empty split or none: exp(-inf) = 0
        if (s < S) wsh[s] = ws;
        sum = __builtin_fmaf(ws, ls[k], sum);
    }
    sum = wave_sum_f32(sum);
    if ((tid & 63) == 0) red[1][wave] = sum;
    __syncthreads();
    const float inv = 1.0f / ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
    // Accumulators: thread (group q, dimension d); group q takes splits q, q + G, ... (G = 256 / the
    // head size rounded up to a power of two), the groups added in order at the end.
    const int G = hd <= 32 ? 8 : hd <= 64 ? 4 : hd <= 128 ? 2 : 1;
    const int per = 256 / G;
    const int q = tid / per, d = tid - q * per;
    float o = 0.0f;
    if (d < hd) {
        int s = q;
        for (; s + 7 * G < S; s += 8 * G) {  // eight splits' loads in flight
            float x[8];
#pragma unroll
            for (int k = 0; k < 8; k++) x[k] = part_acc(a, th, s + k * G)[d];
#pragma unroll
            for (int k = 0; k < 8; k++) o = __builtin_fmaf(wsh[s + k * G], x[k], o);
        }
        for (; s < S; s += G) o = __builtin_fmaf(wsh[s], part_acc(a, th, s)[d], o);
    }
    osh[q][d] = o;
    __syncthreads();
    if (q == 0 && d < hd) {
        for (int k = 1; k < G; k++) o += osh[k][d];
        TQ* orow = static_cast<TQ*>(a.out) + t * a.os + static_cast<int64_t>(h) * hd;
        orow[d] = from_f32<TQ>(o * inv);
    }
}

template <typename TQ, int HDP, int HB>
void launch_hb(neko_hip_ctx* ctx, const AttnArgs& a, dim3 grid, bool vec, bool pf) {
    const dim3 block(64 * kAttnWaves);
    if (!vec) hipLaunchKernelGGL((attn_kernel<TQ, HDP, false, kAttnWaves, HB, false>), grid, block, 0, ctx->stream, a);
    else if (pf) hipLaunchKernelGGL((attn_kernel<TQ, HDP, true, kAttnWaves, HB, true>), grid, block, 0, ctx->stream, a);
    else hipLaunchKernelGGL((attn_kernel<TQ, HDP, true, kAttnWaves, HB, false>), grid, block, 0, ctx->stream, a);
}

template <typename TQ, int HDP>
int launch_hdp(neko_hip_ctx* ctx, const char* what, const AttnArgs& a, bool vec, int64_t items, bool one_head) {
    const dim3 grid(static_cast<uint32_t>(items));
    // The prefetching form where a wave has more than one step (measured: 4096-position decode, one
    // step per wave, 12.7 us without and 15.5 with it; 32768 positions 56.3 -> 49.6 us, the 2048- and
    // 8192-token prefills 6% faster).
    const int step = 8 * (512 / HDP);
    const bool pf = a.split_keys > static_cast<int64_t>(kAttnWaves) * step;
    if (one_head) launch_hb<TQ, HDP, 1>(ctx, a, grid, vec, pf);
    else launch_hb<TQ, HDP, kAttnHeads>(ctx, a, grid, vec, pf);
    if (int rc = after_launch(ctx, what)) return rc;
    if (a.splits == 1) return NEKO_OK;
    hipLaunchKernelGGL((attn_merge_kernel<TQ>), dim3(static_cast<uint32_t>(a.T * a.n_head)), dim3(256), 0, ctx->stream, a);
    return after_launch(ctx, what);
}

template <typename TQ>
int launch_typed(neko_hip_ctx* ctx, const char* what, const AttnArgs& a, bool vec, int64_t items, bool one_head) {
    if (a.hd <= 64) return launch_hdp<TQ, 64>(ctx, what, a, vec, items, one_head);
    if (a.hd <= 128) return launch_hdp<TQ, 128>(ctx, what, a, vec, items, one_head);
    return launch_hdp<TQ, 256>(ctx, what, a, vec, items, one_head);
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" int neko_hip_attention(neko_hip_ctx* ctx, const void* q, int64_t q_stride, const uint16_t* k_cache,
                                  const uint16_t* v_cache, void* out, int64_t out_stride, int64_t T, int n_head, int n_kv,
                                  int hd, int64_t pos0, float scale, int dtype) {
    const char* what = "neko_hip_attention";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, T >= 0 && pos0 >= 0 && n_head > 0 && n_kv > 0 && n_head % n_kv == 0,
                 "%s: bad shape T=%lld pos0=%lld n_head=%d n_kv=%d (n_head a multiple of n_kv)", what, (long long)T,
                 (long long)pos0, n_head, n_kv);
    NEKO_REQUIRE(ctx, hd >= 2 && hd <= 256 && hd % 2 == 0, "%s: head size %d (even, 2..256)", what, hd);
    if (T == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, q && k_cache && v_cache && out, "%s: null pointer", what);
    const int64_t width = static_cast<int64_t>(n_head) * hd;
    NEKO_REQUIRE(ctx, q_stride >= width && out_stride >= width, "%s: q / out row strides (%lld, %lld) below n_head*hd = %lld",
                 what, (long long)q_stride, (long long)out_stride, (long long)width);
    NEKO_REQUIRE(ctx, pos0 <= (int64_t(1) << 40) && T <= (int64_t(1) << 31), "%s: T=%lld / pos0=%lld too large", what,
                 (long long)T, (long long)pos0);
    const size_t esz = dtype_size(dtype);
    const int64_t kvw = static_cast<int64_t>(n_kv) * hd;
    NEKO_REQUIRE(ctx, pos0 + T <= (int64_t(1) << 62) / (kvw * 2), "%s: caches of %lld rows x %lld halves span more "
                 "than 2^62 bytes", what, (long long)(pos0 + T), (long long)kvw);
    const size_t sq = rows_span(T, width, q_stride, esz), so = rows_span(T, width, out_stride, esz);
    const size_t sc = static_cast<size_t>((pos0 + T) * kvw) * 2;
    NEKO_REQUIRE(ctx, sq != 0 && so != 0, "%s: q / out rows span more than 2^62 bytes", what);
    NEKO_REQUIRE(ctx, !overlaps(out, so, q, sq) && !overlaps(out, so, k_cache, sc) && !overlaps(out, so, v_cache, sc),
                 "%s: out may not overlap q or the caches", what);
    AttnArgs a{};
    a.q = q;
    a.qs = q_stride;
    a.kc = k_cache;
    a.vc = v_cache;
    a.kvw = kvw;
    a.out = out;
    a.os = out_stride;
    a.T = T;
    a.pos0 = pos0;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.group = n_head / n_kv;
    // One query head per item where the K and V rows are few (their re-reads by the group's heads stay
    // in L2) and the launch would otherwise be short of waves; else up to four heads share each load.
    const int64_t kv_bytes = (pos0 + T) * static_cast<int64_t>(n_kv) * hd * 4;
    const bool one_head = T * n_kv * ((a.group + kAttnHeads - 1) / kAttnHeads) * kAttnWaves < kAttnTargetWaves &&
                          kv_bytes <= kAttnOneHeadBytes;
    const int hb_size = one_head ? 1 : kAttnHeads;
    a.hblocks = (a.group + hb_size - 1) / hb_size;
    a.hd = hd;
    a.scale = scale;
    // Split the keys when tokens x kv heads x head blocks leave the chip short of waves (each split at
    // least one 64-key step per wave).
    const int64_t base = T * n_kv * a.hblocks;
    const int64_t keys = pos0 + T;  // the longest row
    const int64_t step = 8 * (512 / (hd <= 64 ? 64 : hd <= 128 ? 128 : 256));  // the kernel's keys per step
    const int64_t steps = (keys + step - 1) / step;
    int64_t splits = 1;
    if (base * kAttnWaves < kAttnTargetWaves) {
        const int64_t want = (kAttnTargetWaves + base * kAttnWaves - 1) / (base * kAttnWaves);
        splits = std::min<int64_t>({want, (steps + kAttnWaves - 1) / kAttnWaves, kAttnMaxSplits});
    }
    a.split_keys = (steps + splits - 1) / splits * step;
    a.splits = static_cast<int>((keys + a.split_keys - 1) / a.split_keys);
    const int64_t items = base * a.splits;
    NEKO_REQUIRE(ctx, items <= 0x7fffffff && T * n_head <= 0x7fffffff, "%s: grid too large", what);
    if (a.splits > 1) {
        void* ws = nullptr;
        const size_t bytes = static_cast<size_t>(T) * n_head * a.splits * (hd + 2) * sizeof(float);
        if (int rc = workspace(ctx, bytes, &ws)) return rc;
        a.part = static_cast<float*>(ws);
    }
    const bool vec = hd % 8 == 0 && aligned(k_cache, 16) && aligned(v_cache, 16);
    return dtype == NEKO_DT_F16 ? launch_typed<half_t>(ctx, what, a, vec, items, one_head)
                                : launch_typed<float>(ctx, what, a, vec, items, one_head);
}
