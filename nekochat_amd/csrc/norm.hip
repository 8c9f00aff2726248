// Row norms for gfx950: LayerNorm (cpu_ops.cpp:483-500), RMSNorm (cpu_ops.cpp:502-511), the
// Granite-4.0-H gated group RMSNorm (granite_model.cpp:278-287), and the residual add + RMSNorm
// (the kAccumulate epilogue, cpu_ops.cpp:123, followed by cpu::rmsNorm, qwen3_model.cpp:264).
//
// Fast path: one 64-wide wavefront per row, persistent. A grid of as many 256-thread workgroups as
// stay resident walks the rows. RMSNorm / LayerNorm waves keep their norm weights in registers for
// all of their rows and issue the 16-byte non-temporal loads of the next row before they reduce the
// current one, so HBM is read once, written once, and always has loads in flight. The f16 gated
// norm, which holds two operands per row, spreads each row over 2-8 waves of one workgroup (two
// 16-byte chunks per lane and operand) where its rows split so, else runs persistent with its weights
// in one LDS copy per workgroup and no second row buffer (three times the resident waves instead);
// the residual add + RMSNorm streams x and delta, writes the sum back over x and the norm to xn.
// With many rows per resident wave (3 or more), RMSNorm and LayerNorm instead cover every row with
// its own wave over the whole grid, which the dispatcher keeps full (plain loads and stores, no
// prefetch): a persistent grid's partial last rounds then cost more than its prefetch saves.
// Rows wider than one wave's registers use four waves per row. Sums are accumulated in double, like
// the reference, and reduced across the wave with DPP and v_readlane (LDS only joins the partial
// sums of multi-wave rows). The norm scale is
// rounded to float exactly where the reference rounds it and the output is (x * s) * w unfused, so
// results match the reference's CPU op bit for bit unless a double sum lands within an ulp of a
// float rounding boundary.
//
// Fallback (any width, alignment or stride): one workgroup per row streaming the row from memory
// once per pass.
#include <cmath>

#include "internal.h"

namespace neko_hip {
namespace {

enum class Norm : int { Rms = 0, Layer = 1, Gated = 2, AddRms = 3 };

// Kinds that stream a second operand row: the gate z (Gated) or the residual delta (AddRms).
constexpr bool has_z(Norm k) { return k == Norm::Gated || k == Norm::AddRms; }

struct NormArgs {
    const void* x;  // input rows (the y operand of the gated norm; in/out residual rows of AddRms)
    int64_t xs;
    const void* z;  // gate rows (gated norm) or delta rows (AddRms)
    int64_t zs;
    void* y;  // output rows
    int64_t ys;
    const float* w;  // gamma / norm weight [groups * C]
    const float* b;  // beta (LayerNorm only)
    int64_t rows;    // logical rows = rows * groups
    int C;           // channels per normalised group
    int groups;
    float eps;
};

// Mamba2 output gate, granite_model.cpp:21: v / (1 + exp(-v)) in float, from silu_lite (device.h):
// the gated norm streams two operands per output and was VALU-limited on MI355X with the longer
// forms; silu_lite's relative error (< 1.3e-6 for |v| <= 20) stays far below the fp16 output's half
// ulp (4.9e-4).
__device__ __forceinline__ float silu_ref(float v) { return silu_lite(v); }

// Norm weights in one LDS copy per workgroup (gated and residual norms: frees registers for resident
// waves) or in every lane's registers (RMSNorm, LayerNorm persistent kernels).
constexpr bool weights_in_lds(Norm k) { return k == Norm::Gated || k == Norm::AddRms; }

// Overlap of a persistent wave's next row: a second row buffer loaded before the current row is
// reduced (RMSNorm, LayerNorm, residual add + RMSNorm), or none (the gated norm, whose rows hold two
// operands: three times the resident waves beat a second buffer).
constexpr bool prefetches(Norm k) { return k != Norm::Gated; }

// RMSNorm / LayerNorm take the one-row-per-wave grid from this many rows per resident persistent wave.
constexpr int64_t kRowRatio = 3;

// Output stores: non-temporal for the plain norms, plain for the gated norm and the residual add +
// RMSNorm (measured at [8192, 2560]: non-temporal 17.1 vs 17.9 us for the persistent RMSNorm, plain
// 29.7 vs 31.3 us for the residual add + RMSNorm, which stores two rows per row). PLAIN: the
// one-row-per-wave kernel, whose plain loads and stores measured faster than non-temporal ones there.
template <Norm K, bool PLAIN = false, typename V>
__device__ __forceinline__ void store_out(V* p, V v) {
    constexpr bool nt = K == Norm::Rms || K == Norm::Layer;
    if constexpr (!PLAIN && nt) store_nt(p, v);
    else *p = v;
}

template <Norm K, typename T>
struct RowPtrs {
    const T* x;
    const T* z;
    T* y;
    const float* w;
    const float* b;
};

template <Norm K, typename T>
__device__ __forceinline__ RowPtrs<K, T> row_ptrs(const NormArgs& a, int64_t r) {
    const int64_t t = a.groups == 1 ? r : r / a.groups;
    const int64_t g = r - t * a.groups;
    const int64_t off = g * a.C;
    RowPtrs<K, T> p;
    p.x = static_cast<const T*>(a.x) + t * a.xs + off;
    p.z = has_z(K) ? static_cast<const T*>(a.z) + t * a.zs + off : nullptr;
    p.y = static_cast<T*>(a.y) + t * a.ys + off;
    p.w = a.w + off;
    p.b = a.b;
    return p;
}

// ------------------------------------------------------------------ register-resident rows
// The row (and the gate operand) of one lane: up to CH 16-byte chunks, chunk j = k * NT + tid.
template <Norm K, typename T, int CH>
struct RowRegs {
    typedef typename Chunk16<T>::V V;
    V x[CH];
    V z[CH];
};

// Row loads: non-temporal, plain in the one-row-per-wave kernel (PLAIN).
template <bool PLAIN = false, typename V>
__device__ __forceinline__ V load_row_chunk(const V* p) {
    if constexpr (!PLAIN) return load_nt(p);
    else return *p;
}

template <Norm K, typename T, int CH, int NT, bool PLAIN = false>
__device__ __forceinline__ void load_row(RowRegs<K, T, CH>& rr, const RowPtrs<K, T>& p, int tid, int nch) {
    typedef typename Chunk16<T>::V V;
    constexpr int N = Chunk16<T>::N;
#pragma unroll
    for (int k = 0; k < CH; k++) {
        const int j = k * NT + tid;
        rr.x[k] = V{};
        rr.z[k] = V{};
        if (j < nch) {
            rr.x[k] = load_row_chunk<PLAIN>(reinterpret_cast<const V*>(p.x + j * N));
            if constexpr (has_z(K)) rr.z[k] = load_row_chunk<PLAIN>(reinterpret_cast<const V*>(p.z + j * N));
        }
    }
}

// AddRms: the row becomes x + delta, added in float and rounded once to T (the residual the
// reference's kAccumulate epilogue leaves, cpu_ops.cpp:123); the norm then reads that rounded row.
template <Norm K, typename T, int CH>
__device__ __forceinline__ void add_residual(RowRegs<K, T, CH>& rr) {
    if constexpr (K == Norm::AddRms) {
#pragma unroll
        for (int k = 0; k < CH; k++)
#pragma unroll
            for (int e = 0; e < Chunk16<T>::N; e++) rr.x[k][e] = from_f32<T>(to_f32(rr.x[k][e]) + to_f32(rr.z[k][e]));
    }
}

// AddRms: writes the updated residual chunks back over x.
template <Norm K, typename T, int CH, int NT, bool PLAIN = false>
__device__ __forceinline__ void store_residual(const RowRegs<K, T, CH>& rr, const RowPtrs<K, T>& p, int tid, int nch) {
    if constexpr (K == Norm::AddRms) {
        typedef typename Chunk16<T>::V V;
        constexpr int N = Chunk16<T>::N;
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int j = k * NT + tid;
            if (j < nch) store_out<K, PLAIN>(reinterpret_cast<V*>(const_cast<T*>(p.x) + j * N), rr.x[k]);
        }
    }
}

// The norm weights (and LayerNorm's beta) of one lane's chunks, as float4 quads: held in registers
// (WL = false), or read at the store from the workgroup's LDS copy of the weight vector (WL = true).
template <Norm K, typename T, int CH, int NT, bool WL>
struct Weights {
    static constexpr int N = Chunk16<T>::N;
    float4v w[CH][N / 4], b[CH][N / 4];

    __device__ __forceinline__ void init(const float* wp, const float* bp, int tid, int nch) {
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int j = k * NT + tid;
#pragma unroll
            for (int q = 0; q < N / 4; q++) {
                w[k][q] = float4v{};
                b[k][q] = float4v{};
                if (j < nch) {
                    w[k][q] = *reinterpret_cast<const float4v*>(wp + j * N + 4 * q);
                    if constexpr (K == Norm::Layer) b[k][q] = *reinterpret_cast<const float4v*>(bp + j * N + 4 * q);
                }
            }
        }
    }
    __device__ __forceinline__ float4v wq(int k, int q) const { return w[k][q]; }
    __device__ __forceinline__ float4v bq(int k, int q) const { return b[k][q]; }
};

template <Norm K, typename T, int CH, int NT>
struct Weights<K, T, CH, NT, true> {
    static constexpr int N = Chunk16<T>::N;
    const float* w;  // LDS: this row group's weights, at this lane's first chunk
    const float* b;

    __device__ __forceinline__ void init(const float* wl, const float* bl, int tid, int) {
        w = wl + tid * N;
        b = bl + tid * N;
    }
    __device__ __forceinline__ float4v wq(int k, int q) const {
        return *reinterpret_cast<const float4v*>(w + k * NT * N + 4 * q);
    }
    __device__ __forceinline__ float4v bq(int k, int q) const {
        return *reinterpret_cast<const float4v*>(b + k * NT * N + 4 * q);
    }
};

// The row in float. Plain norms convert from the loaded halves on every use (cheaper than holding a
// float copy in registers); the gated norm evaluates y * silu(z) once and keeps it (evaluating it again
// at the store doubles the silu work). Lanes past the row end hold zeros, which add nothing to the
// sums.
template <Norm K, typename T, int CH>
struct RowVals {
    static constexpr int N = Chunk16<T>::N;
    static constexpr bool kKeep = K == Norm::Gated;
    float f[kKeep ? CH : 1][kKeep ? N : 1];
    const RowRegs<K, T, CH>* rr;

    __device__ __forceinline__ void init(const RowRegs<K, T, CH>& regs) {
        rr = &regs;
        if constexpr (kKeep) {
#pragma unroll
            for (int k = 0; k < CH; k++)
#pragma unroll
                for (int e = 0; e < N; e++) f[k][e] = to_f32(regs.x[k][e]) * silu_ref(to_f32(regs.z[k][e]));
        }
    }
    __device__ __forceinline__ float operator()(int k, int e) const {
        if constexpr (kKeep) return f[k][e];
        else return to_f32(rr->x[k][e]);
    }
};

// Squares of f16 values, and of the f32 values the f32 ABI passes, are exact in double, so
// fma(d, d, s) equals the reference's s += d * d.
template <int CH, int N, typename F>
__device__ __forceinline__ double sum_squares(const F& f) {
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < CH; k++)
#pragma unroll
        for (int e = 0; e < N; e++) {
            const double d = static_cast<double>(f(k, e));
            ss = __builtin_fma(d, d, ss);
        }
    return ss;
}

template <int CH, int N, typename F>
__device__ __forceinline__ double sum_values(const F& f) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < CH; k++)
#pragma unroll
        for (int e = 0; e < N; e++) s += static_cast<double>(f(k, e));
    return s;
}

// Sum of (x - mean)^2 over valid chunks; the product is rounded before the add, as in the reference.
template <int CH, int N, int NT, typename F>
__device__ __forceinline__ double sum_centered(const F& f, double mean, int tid, int nch) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < CH; k++) {
        const int j = k * NT + tid;
#pragma unroll
        for (int e = 0; e < N; e++) {
            const double d = static_cast<double>(f(k, e)) - mean;
            if (j < nch) s += d * d;
        }
    }
    return s;
}

// Output chunk k: (x - mean) * scale * gamma + beta, or x * scale * w, rounded once.
template <Norm K, typename T, int CH, typename F, typename W>
__device__ __forceinline__ typename Chunk16<T>::V out_chunk(const F& f, int k, float scale, float mean_f, const W& wt) {
    constexpr int N = Chunk16<T>::N;
    typename Chunk16<T>::V out;
#pragma unroll
    for (int q = 0; q < N / 4; q++) {
        const float4v w = wt.wq(k, q);
        float4v b{};
        if constexpr (K == Norm::Layer) b = wt.bq(k, q);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = 4 * q + i;
            float v;
            if constexpr (K == Norm::Layer) v = (f(k, e) - mean_f) * scale * w[i] + b[i];
            else v = f(k, e) * scale * w[i];
            out[e] = from_f32<T>(v);
        }
    }
    return out;
}

template <Norm K, typename T, int CH, int NT, bool PLAIN = false, typename F, typename W>
__device__ __forceinline__ void store_row(T* y, const F& f, float scale, float mean_f, const W& wt, int tid, int nch) {
    typedef typename Chunk16<T>::V V;
    constexpr int N = Chunk16<T>::N;
#pragma unroll
    for (int k = 0; k < CH; k++) {
        const int j = k * NT + tid;
        if (j >= nch) continue;
        store_out<K, PLAIN>(reinterpret_cast<V*>(y + j * N), out_chunk<K, T, CH>(f, k, scale, mean_f, wt));
    }
}

// One wavefront per row, persistent: wave w handles rows w, w + nw, ... (nw = waves in the grid),
// keeps the weights in registers (or its workgroup's LDS copy) across rows and loads the next row
// while it normalises this one. Every row of a wave shares one group index (the host makes nw a
// multiple of groups, or gives each wave at most one row). With WL the dynamic LDS holds the
// groups * C weights (then C betas for LayerNorm). ROW: the grid covers every row, one per wave,
// with plain loads and stores and no prefetch registers (the form for many rows per resident wave).
template <Norm K, typename T, int CH, bool WL, bool ROW = false, bool PF = !ROW && prefetches(K)>
__global__ __launch_bounds__(256) void norm_wave_kernel(NormArgs a) {
    constexpr int N = Chunk16<T>::N;
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    extern __shared__ float4v wlds[];
    if constexpr (WL) {
        // Every wave reaches this barrier before any may leave.
        const int nq = a.groups * a.C / 4;
        float4v* wl = wlds;
        for (int i = threadIdx.x; i < nq; i += 256) wl[i] = reinterpret_cast<const float4v*>(a.w)[i];
        if constexpr (K == Norm::Layer)
            for (int i = threadIdx.x; i < a.C / 4; i += 256) wl[nq + i] = reinterpret_cast<const float4v*>(a.b)[i];
        __syncthreads();
    }
    // readfirstlane tells the compiler the row index is wave-uniform, so row pointers stay in SGPRs.
    int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= a.rows) return;  // wave-uniform
    const int nch = a.C / N;
    const RowPtrs<K, T> p0 = row_ptrs<K, T>(a, r);
    Weights<K, T, CH, kWave, WL> wt;
    if constexpr (WL) {
        const float* wl = reinterpret_cast<const float*>(wlds);
        wt.init(wl + (p0.w - a.w), wl + a.groups * a.C, lane, nch);
    } else {
        wt.init(p0.w, p0.b, lane, nch);
    }

    RowRegs<K, T, CH> cur, nxt;
    load_row<K, T, CH, kWave, ROW>(cur, p0, lane, nch);
    for (; r < a.rows; r += nw) {
        const bool more = r + nw < a.rows;
        if (PF && more) load_row<K, T, CH, kWave, ROW>(nxt, row_ptrs<K, T>(a, r + nw), lane, nch);
        add_residual(cur);
        RowVals<K, T, CH> f;
        f.init(cur);
        float scale, mean_f = 0.0f;
        if constexpr (K == Norm::Layer) {
            const double mean = wave_sum_f64(sum_values<CH, N>(f)) / a.C;
            const double var = wave_sum_f64(sum_centered<CH, N, kWave>(f, mean, lane, nch)) / a.C;
            scale = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
            mean_f = static_cast<float>(mean);
        } else {
            const double ss = wave_sum_f64(sum_squares<CH, N>(f));
            scale = static_cast<float>(1.0 / sqrt(ss / a.C + static_cast<double>(a.eps)));
        }
        const RowPtrs<K, T> pc = row_ptrs<K, T>(a, r);
        store_row<K, T, CH, kWave, ROW>(pc.y, f, scale, mean_f, wt, lane, nch);
        store_residual<K, T, CH, kWave, ROW>(cur, pc, lane, nch);
        if (PF && more) cur = nxt;
        else if (more) load_row<K, T, CH, kWave, ROW>(cur, row_ptrs<K, T>(a, r + nw), lane, nch);
    }
}

// ------------------------------------------------------------------ one round
// RMSNorm / LayerNorm when every row fits in one round of resident waves: wave w of nw takes rows
// w, w + nw, ... (R of them, nw * R >= rows) and requests all of their bytes first, through
// range-checked buffer resources (lanes past the row end, and rows past the last, read zeros and drop
// their stores, so no load sits under a branch). Then each workgroup stages the norm weights (and
// LayerNorm's beta) in LDS -- quad q of 16-byte chunk j at q * nch + j, so a wave's reads of one
// quad are consecutive -- and meets at one barrier: its reads all land before any of its writes.
// Each wave then normalises and stores (non-temporal) its rows, with the arithmetic of
// norm_wave_kernel. Measured at [8192, 2560] f16: 15.0 us against 17.1 for the persistent kernel and
// 16.7 for a copy of the same bytes in this shape without the barrier.
template <typename T, int CH>
struct RoundWeights {
    static constexpr int N = Chunk16<T>::N;
    const float4v* w;  // LDS: weight quads, then beta quads at N / 4 * nch
    int j0;            // this lane's first chunk
    int nch;
    __device__ __forceinline__ int chunk(int k) const { return min(j0 + k * kWave, nch - 1); }
    __device__ __forceinline__ float4v wq(int k, int q) const { return w[q * nch + chunk(k)]; }
    __device__ __forceinline__ float4v bq(int k, int q) const { return w[(N / 4 + q) * nch + chunk(k)]; }
};

template <Norm K, typename T, int CH, int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void norm_round_kernel(NormArgs a) {
    static_assert(K != Norm::Gated, "plain norms and the residual add + RMSNorm");
    constexpr int N = Chunk16<T>::N;
    constexpr bool kAdd = K == Norm::AddRms;
    // Stores: non-temporal for the plain norms; plain for the residual add + RMSNorm, which writes two
    // rows per row (measured at [8192, 2560]: 28.9 us plain, 30.8 non-temporal).
    constexpr bool kNt = !kAdd;
    typedef typename Chunk16<T>::V V;
    extern __shared__ float4v rlds[];
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = a.C / N;
    const uint32_t row_bytes = static_cast<uint32_t>(a.C) * sizeof(T);
    V x[R][CH], z[kAdd ? R : 1][kAdd ? CH : 1];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int64_t row = w + r * nw;
        const bool in = row < a.rows;
        const BufRes res = buf_res(static_cast<const T*>(a.x) + (in ? row : 0) * a.xs, in ? row_bytes : 0u);
#pragma unroll
        for (int k = 0; k < CH; k++) x[r][k] = buf_load16<true, V>(res, static_cast<uint32_t>(k * kWave + lane) * 16u);
        if constexpr (kAdd) {
            const BufRes rz = buf_res(static_cast<const T*>(a.z) + (in ? row : 0) * a.zs, in ? row_bytes : 0u);
#pragma unroll
            for (int k = 0; k < CH; k++) z[r][k] = buf_load16<true, V>(rz, static_cast<uint32_t>(k * kWave + lane) * 16u);
        }
    }
    {
        const int nq = nch * (N / 4);
        const float4v* wg = reinterpret_cast<const float4v*>(a.w);
        for (int i = threadIdx.x; i < nq; i += 256) rlds[(i % (N / 4)) * nch + i / (N / 4)] = wg[i];
        if constexpr (K == Norm::Layer) {
            const float4v* bg = reinterpret_cast<const float4v*>(a.b);
            for (int i = threadIdx.x; i < nq; i += 256) rlds[(N / 4 + i % (N / 4)) * nch + i / (N / 4)] = bg[i];
        }
    }
    __syncthreads();
    const RoundWeights<T, CH> wt{rlds, lane, nch};
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int64_t row = w + r * nw;
        if (row >= a.rows) break;  // wave-uniform
        auto f = [&](int k, int e) __attribute__((always_inline)) -> float { return to_f32(x[r][k][e]); };
        float scale, mean_f = 0.0f;
        if constexpr (kAdd) {
            // The residual x + delta, rounded once to T (cpu_ops.cpp:123), is what the norm reads; its
            // squares are summed as each value is formed.
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < CH; k++)
#pragma unroll
                for (int e = 0; e < N; e++) {
                    x[r][k][e] = from_f32<T>(to_f32(x[r][k][e]) + to_f32(z[r][k][e]));
                    const double d = static_cast<double>(to_f32(x[r][k][e]));
                    ss = __builtin_fma(d, d, ss);
                }
            ss = wave_sum_f64(ss);
            scale = static_cast<float>(1.0 / sqrt(ss / a.C + static_cast<double>(a.eps)));
        } else if constexpr (K == Norm::Layer) {
            const double mean = wave_sum_f64(sum_values<CH, N>(f)) / a.C;
            const double var = wave_sum_f64(sum_centered<CH, N, kWave>(f, mean, lane, nch)) / a.C;
            scale = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
            mean_f = static_cast<float>(mean);
        } else {
            const double ss = wave_sum_f64(sum_squares<CH, N>(f));
            scale = static_cast<float>(1.0 / sqrt(ss / a.C + static_cast<double>(a.eps)));
        }
        const BufRes res = buf_res(static_cast<T*>(a.y) + row * a.ys, row_bytes);
        const BufRes rx = buf_res(static_cast<const T*>(a.x) + row * a.xs, kAdd ? row_bytes : 0u);
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const uint32_t off = static_cast<uint32_t>(k * kWave + lane) * 16u;
            if constexpr (kAdd) buf_store16<kNt>(rx, off, x[r][k]);  // the residual back over x
            buf_store16<kNt>(res, off, out_chunk<K, T, CH>(f, k, scale, mean_f, wt));
        }
    }
}

// WPR wavefronts per row (one row per workgroup), CH chunks per lane: rows wider than one wave's
// registers (four waves, non-temporal loads), and the f16 gated norm wherever its rows split evenly
// into two chunks per lane over 2-8 waves (PLAIN loads): at [16384, 3072] three waves per row take
// 47.9 us against 51.6 for the persistent one-wave kernel (every output bit-identical), at eight
// waves per SIMD and without a second row buffer -- the waves of the other rows are the overlap.
// (Plain loads beat non-temporal ones there by 0.7 us, plain stores non-temporal ones by 4 us; two
// waves of three chunks took 50.5, six of one 52.9, one wave of six over the whole grid 51.0.) The
// partial sums meet in LDS.
template <Norm K, typename T, int CH, int WPR = 4, bool PLAIN = false>
__global__ __launch_bounds__(WPR * kWave) void norm_wide_kernel(NormArgs a) {
    constexpr int N = Chunk16<T>::N;
    constexpr int NT = WPR * kWave;
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int nch = a.C / N;
    const RowPtrs<K, T> p = row_ptrs<K, T>(a, r);
    RowRegs<K, T, CH> rr;
    load_row<K, T, CH, NT, PLAIN>(rr, p, tid, nch);
    add_residual(rr);
    Weights<K, T, CH, NT, false> wt;
    wt.init(p.w, p.b, tid, nch);
    RowVals<K, T, CH> f;
    f.init(rr);

    __shared__ double part[2][WPR];
    auto block_total = [&](double v, int slot) -> double {
        v = wave_sum_f64(v);
        if ((tid & 63) == 0) part[slot][wave] = v;
        __syncthreads();
        if constexpr (WPR == 4) return (part[slot][0] + part[slot][1]) + (part[slot][2] + part[slot][3]);
        double s = part[slot][0];
#pragma unroll
        for (int i = 1; i < WPR; i++) s += part[slot][i];
        return s;
    };
    float scale, mean_f = 0.0f;
    if constexpr (K == Norm::Layer) {
        const double mean = block_total(sum_values<CH, N>(f), 0) / a.C;
        const double var = block_total(sum_centered<CH, N, NT>(f, mean, tid, nch), 1) / a.C;
        scale = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
        mean_f = static_cast<float>(mean);
    } else {
        const double ss = block_total(sum_squares<CH, N>(f), 0);
        scale = static_cast<float>(1.0 / sqrt(ss / a.C + static_cast<double>(a.eps)));
    }
    store_row<K, T, CH, NT>(p.y, f, scale, mean_f, wt, tid, nch);
    store_residual<K, T, CH, NT>(rr, p, tid, nch);
}

// ------------------------------------------------------------------ generic rows
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
    v = wave_sum_f64(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const double s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

template <Norm K, typename T>
__device__ __forceinline__ float gen_value(const RowPtrs<K, T>& p, int c) {
    if constexpr (K == Norm::Gated) return to_f32(p.x[c]) * silu_ref(to_f32(p.z[c]));
    else return to_f32(p.x[c]);
}

template <Norm K, typename T>
__global__ __launch_bounds__(256) void norm_rows_generic(NormArgs a) {
    __shared__ double red[4];
    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
        const RowPtrs<K, T> p = row_ptrs<K, T>(a, r);
        float scale, mean_f = 0.0f;
        if constexpr (K == Norm::Layer) {
            double s1 = 0.0;
            for (int c = threadIdx.x; c < a.C; c += 256) s1 += static_cast<double>(gen_value<K, T>(p, c));
            const double mean = block_sum_f64(s1, red) / a.C;
            double s2 = 0.0;
            for (int c = threadIdx.x; c < a.C; c += 256) {
                const double d = static_cast<double>(gen_value<K, T>(p, c)) - mean;
                s2 += d * d;
            }
            const double var = block_sum_f64(s2, red) / a.C;
            scale = static_cast<float>(1.0 / sqrt(var + static_cast<double>(a.eps)));
            mean_f = static_cast<float>(mean);
        } else {
            double ss = 0.0;
            for (int c = threadIdx.x; c < a.C; c += 256) {
                if constexpr (K == Norm::AddRms) {
                    // The residual sum is written back at once; the store pass below reads the value
                    // this same thread wrote.
                    const T s = from_f32<T>(to_f32(p.x[c]) + to_f32(p.z[c]));
                    const_cast<T*>(p.x)[c] = s;
                }
                const double d = static_cast<double>(gen_value<K, T>(p, c));
                ss += d * d;
            }
            scale = static_cast<float>(1.0 / sqrt(block_sum_f64(ss, red) / a.C + static_cast<double>(a.eps)));
        }
        // Separate loops per pass: the output may alias the input, so every read of this row by
        // any thread precedes the barrier inside block_sum_f64 above.
        for (int c = threadIdx.x; c < a.C; c += 256) {
            const float v = gen_value<K, T>(p, c);
            float o;
            if constexpr (K == Norm::Layer) o = (v - mean_f) * scale * p.w[c] + p.b[c];
            else o = v * scale * p.w[c];
            p.y[c] = from_f32<T>(o);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ dispatch
typedef void (*NormKernel)(NormArgs);

template <Norm K, typename T, bool WL, bool ROW>
NormKernel pick_wave(int CH) {
    switch (CH) {
        case 1: return norm_wave_kernel<K, T, 1, WL, ROW>;
        case 2: return norm_wave_kernel<K, T, 2, WL, ROW>;
        case 3: return norm_wave_kernel<K, T, 3, WL, ROW>;
        case 4: return norm_wave_kernel<K, T, 4, WL, ROW>;
        case 5: return norm_wave_kernel<K, T, 5, WL, ROW>;
        case 6: return norm_wave_kernel<K, T, 6, WL, ROW>;
        case 8: return norm_wave_kernel<K, T, 8, WL, ROW>;
    }
    return nullptr;
}

template <Norm K, typename T>
NormKernel pick_wide(int CH) {
    switch (CH) {
        case 4: return norm_wide_kernel<K, T, 4>;
        case 8: return norm_wide_kernel<K, T, 8>;
    }
    return nullptr;
}

// The f16 gated norm over WPR waves per row, two chunks per lane (plain loads).
NormKernel pick_gated_split(int WPR) {
    switch (WPR) {
        case 2: return norm_wide_kernel<Norm::Gated, half_t, 2, 2, true>;
        case 3: return norm_wide_kernel<Norm::Gated, half_t, 2, 3, true>;
        case 4: return norm_wide_kernel<Norm::Gated, half_t, 2, 4, true>;
        case 5: return norm_wide_kernel<Norm::Gated, half_t, 2, 5, true>;
        case 6: return norm_wide_kernel<Norm::Gated, half_t, 2, 6, true>;
        case 7: return norm_wide_kernel<Norm::Gated, half_t, 2, 7, true>;
        case 8: return norm_wide_kernel<Norm::Gated, half_t, 2, 8, true>;
    }
    return nullptr;
}

// The one-row-per-wave form exists for the plain norms (RMSNorm, LayerNorm) with weights in
// registers; the gated and residual norms measured no gain from it.
constexpr bool has_row_form(Norm k) { return k == Norm::Rms || k == Norm::Layer; }

// The one-round kernel for R rows of CH chunks per lane, instantiated where it compiles within 128
// VGPRs (four waves per SIMD) without spills: RMSNorm while a wave's rows take at most 60 data
// registers (CH * R <= 15 16-byte chunks), the residual add + RMSNorm (two operand rows) up to 10,
// LayerNorm -- whose two passes keep the row's values widened to double between them -- up to 4.
constexpr int round_max_chunks(Norm k) { return k == Norm::Layer ? 4 : k == Norm::AddRms ? 10 : 15; }
// Up to three rows per wave: four (16384 rows of 1536 halves) measured 3% slower than one row per wave
// over the whole grid.
constexpr int kRoundMaxRows = 3;

template <Norm K, typename T, int CH>
NormKernel pick_round_r(int R) {
    constexpr int M = round_max_chunks(K);
    switch (R) {
        case 1: if constexpr (CH <= M) return norm_round_kernel<K, T, CH, 1>; break;
        case 2: if constexpr (2 * CH <= M) return norm_round_kernel<K, T, CH, 2>; break;
        case 3: if constexpr (3 * CH <= M) return norm_round_kernel<K, T, CH, 3>; break;
    }
    return nullptr;
}

template <Norm K, typename T>
NormKernel pick_round(int CH, int R) {
    switch (CH) {
        case 1: return pick_round_r<K, T, 1>(R);
        case 2: return pick_round_r<K, T, 2>(R);
        case 3: return pick_round_r<K, T, 3>(R);
        case 4: return pick_round_r<K, T, 4>(R);
        case 5: return pick_round_r<K, T, 5>(R);
        case 6: return pick_round_r<K, T, 6>(R);
        case 7: return pick_round_r<K, T, 7>(R);
        case 8: return pick_round_r<K, T, 8>(R);
    }
    return nullptr;
}

template <Norm K>
NormKernel pick(int dtype, int W, int CH, bool wl, bool row = false) {
    const bool h = dtype == NEKO_DT_F16;
    if (W == 0) return h ? norm_rows_generic<K, half_t> : norm_rows_generic<K, float>;
    if (W == 1) {
        if constexpr (has_row_form(K))
            if (row && !wl) return h ? pick_wave<K, half_t, false, true>(CH) : pick_wave<K, float, false, true>(CH);
        if (wl) return h ? pick_wave<K, half_t, true, false>(CH) : pick_wave<K, float, true, false>(CH);
        return h ? pick_wave<K, half_t, false, false>(CH) : pick_wave<K, float, false, false>(CH);
    }
    return h ? pick_wide<K, half_t>(CH) : pick_wide<K, float>(CH);
}

constexpr size_t kMaxWeightLds = 32768;  // bytes of weights one workgroup may stage in LDS

int64_t gcd64(int64_t a, int64_t b) {
    while (b) {
        const int64_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

int launch_norm(neko_hip_ctx* ctx, Norm kind, const NormArgs& a, int dtype, const char* what) {
    const size_t esz = dtype_size(dtype);
    const int N = static_cast<int>(16 / esz);
    // The register paths load 16-byte chunks of every operand row and 16-byte weight vectors.
    bool vec = a.C % N == 0 && aligned(a.x, 16) && aligned(a.y, 16) && aligned(a.w, 16) && (a.xs * esz) % 16 == 0 &&
               (a.ys * esz) % 16 == 0;
    if (kind == Norm::Gated || kind == Norm::AddRms) vec = vec && aligned(a.z, 16) && (a.zs * esz) % 16 == 0;
    if (kind == Norm::Layer) vec = vec && aligned(a.b, 16);
    int W = 0, CH = 0;
    if (vec) {
        const int nch = a.C / N;
        if (nch <= kWave * 8) {
            W = 1;
            CH = (nch + kWave - 1) / kWave;
            if (CH == 7) CH = 8;
        } else if (nch <= 4 * kWave * 8) {
            W = 4;
            CH = (nch + 4 * kWave - 1) / (4 * kWave) <= 4 ? 4 : 8;
        }
    }
    // Weights staged in LDS: groups * C floats (+ C betas), when they fit and the kind asks for it.
    const size_t lds = (static_cast<size_t>(a.groups) * a.C + (kind == Norm::Layer ? a.C : 0)) * sizeof(float);
    const bool wl = W == 1 && weights_in_lds(kind) && lds <= kMaxWeightLds && (kind != Norm::Layer || aligned(a.b, 16));
    // The f16 gated norm whose rows split into two chunks per lane over 2-8 waves: one row per
    // workgroup of that many waves.
    if (kind == Norm::Gated && vec && dtype == NEKO_DT_F16 && a.C / N % (2 * kWave) == 0) {
        const int wpr = a.C / N / (2 * kWave);
        if (wpr >= 2 && wpr <= 8) {
            if (a.rows > 0x7fffffff)
                return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: %lld rows exceed one launch", what, (long long)a.rows);
            hipLaunchKernelGGL(pick_gated_split(wpr), dim3(static_cast<uint32_t>(a.rows)), dim3(wpr * kWave), 0, ctx->stream,
                               a);
            return after_launch(ctx, what);
        }
    }
    NormKernel k = nullptr;
    switch (kind) {
        case Norm::Rms: k = pick<Norm::Rms>(dtype, W, CH, wl); break;
        case Norm::Layer: k = pick<Norm::Layer>(dtype, W, CH, wl); break;
        case Norm::Gated: k = pick<Norm::Gated>(dtype, W, CH, wl); break;
        case Norm::AddRms: k = pick<Norm::AddRms>(dtype, W, CH, wl); break;
    }
    if (!k) return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: no kernel for C=%d", what, a.C);
    if (W == 1 && kind != Norm::Gated && a.groups == 1) {
        // Up to three rows per wave in one round of four waves per SIMD: R = the rows per wave that
        // round needs (measured at 2560 halves: 4096 rows R = 1 9.3 us against 11.0 for the
        // one-row-per-wave grid, 8192 rows R = 2 15.0 against 17.1 persistent, 12288 rows R = 3 22.8
        // against 23.3; at 8192 rows R = 1 over the whole grid at eight waves per SIMD took 16.9).
        const int64_t round = static_cast<int64_t>(ctx->cu_count > 0 ? ctx->cu_count : 256) * 16;
        const int64_t R = (a.rows + round - 1) / round;
        NormKernel kr = nullptr;
        if (R <= kRoundMaxRows) {
            const bool h = dtype == NEKO_DT_F16;
            const int r = static_cast<int>(R);
            switch (kind) {
                case Norm::Rms: kr = h ? pick_round<Norm::Rms, half_t>(CH, r) : pick_round<Norm::Rms, float>(CH, r); break;
                case Norm::Layer: kr = h ? pick_round<Norm::Layer, half_t>(CH, r) : pick_round<Norm::Layer, float>(CH, r); break;
                case Norm::AddRms:
                    kr = h ? pick_round<Norm::AddRms, half_t>(CH, r) : pick_round<Norm::AddRms, float>(CH, r);
                    break;
                default: break;
            }
        }
        if (kr) {
            const size_t rl = static_cast<size_t>(a.C) * sizeof(float) * (kind == Norm::Layer ? 2 : 1);
            const int64_t waves = (a.rows + R - 1) / R;
            const int64_t rblocks = (waves + 3) / 4;
            // Rows w + r * nw (nw = 4 * rblocks, r < R) cover every row once: nw * R >= rows.
            hipLaunchKernelGGL(kr, dim3(static_cast<uint32_t>(rblocks)), dim3(256), rl, ctx->stream, a);
            return after_launch(ctx, what);
        }
    }
    int64_t blocks;
    if (W == 1 && has_row_form(kind) && !wl) {
        // Many rows per resident wave: one row per wave over the whole grid, which the dispatcher keeps
        // full, instead of persistent waves (measured at 2560 and 1536 halves: 16384 and 32768 rows
        // 7-12% faster, 8192 rows of 2560 -- 2.7 per resident wave -- 5% slower).
        const int64_t resident = static_cast<int64_t>(ctx->cu_count > 0 ? ctx->cu_count : 256) * 4 *
                                 resident_blocks_per_cu(reinterpret_cast<const void*>(k), 256, 0);
        if (a.rows >= kRowRatio * resident) {
            NormKernel kr = nullptr;
            switch (kind) {
                case Norm::Rms: kr = pick<Norm::Rms>(dtype, W, CH, wl, true); break;
                case Norm::Layer: kr = pick<Norm::Layer>(dtype, W, CH, wl, true); break;
                default: break;
            }
            if (kr) {
                const int64_t rblocks = (a.rows + 3) / 4;
                if (rblocks > 0x7fffffff)
                    return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: %lld rows exceed one launch", what, (long long)a.rows);
                hipLaunchKernelGGL(kr, dim3(static_cast<uint32_t>(rblocks)), dim3(256), 0, ctx->stream, a);
                return after_launch(ctx, what);
            }
        }
    }
    if (W == 1) {
        // Persistent waves: as many workgroups as stay resident together. A wave that handles several
        // rows must see one group index, so the wave count is then a multiple of groups.
        const int64_t need = (a.rows + 3) / 4;
        blocks = persistent_grid(ctx, reinterpret_cast<const void*>(k), 256, need, wl ? lds : 0);
        if (blocks < need) {
            const int64_t m = a.groups / gcd64(a.groups, 4);
            blocks = blocks / m * m;
            if (blocks == 0) blocks = m;
        }
    } else if (W == 4) {
        blocks = a.rows;
    } else {
        blocks = a.rows < 65536 ? a.rows : 65536;
    }
    if (blocks > 0x7fffffff) return fail(ctx, NEKO_ERR_UNSUPPORTED, "%s: %lld rows exceed one launch", what, (long long)a.rows);
    hipLaunchKernelGGL(k, dim3(static_cast<uint32_t>(blocks)), dim3(256), wl ? lds : 0, ctx->stream, a);
    return after_launch(ctx, what);
}

int check_rows(neko_hip_ctx* ctx, const char* what, int64_t rows, int64_t C, int64_t stride, const char* name) {
    NEKO_REQUIRE(ctx, stride >= C, "%s: %s stride %lld < row width %lld", what, name, (long long)stride, (long long)C);
    NEKO_REQUIRE(ctx, rows_span(rows, C, stride, 4) != 0, "%s: %s rows span more than 2^62 bytes", what, name);
    return NEKO_OK;
}

// Rows read at `in` and written at `out`: the same rows (in place) or disjoint (allow_same = false:
// disjoint only). Persistent waves load a later row while storing the current one, so any partial
// overlap would race.
int check_alias(neko_hip_ctx* ctx, const char* what, const void* in, int64_t in_stride, const char* in_name, const void* out,
                int64_t out_stride, const char* out_name, int64_t rows, int64_t C, int dtype, bool allow_same = true) {
    const size_t esz = dtype_size(dtype);
    const size_t si = rows_span(rows, C, in_stride, esz), so = rows_span(rows, C, out_stride, esz);
    if (allow_same)
        NEKO_REQUIRE(ctx, same_or_disjoint(in, in_stride, out, out_stride, si, so),
                     "%s: %s and %s overlap without being the same rows (same pointer and stride)", what, in_name, out_name);
    else
        NEKO_REQUIRE(ctx, !overlaps(in, si, out, so), "%s: %s may not overlap %s", what, out_name, in_name);
    return NEKO_OK;
}

}  // namespace
}  // namespace neko_hip

using namespace neko_hip;

extern "C" {

int neko_hip_layernorm(neko_hip_ctx* ctx, const void* x, int64_t x_stride, void* y, int64_t y_stride, const float* gamma,
                       const float* beta, int64_t rows, int64_t C, float eps, int dtype) {
    const char* what = "neko_hip_layernorm";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && C > 0 && C <= 0x7fffffff, "%s: bad shape rows=%lld C=%lld", what, (long long)rows,
                 (long long)C);
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, x && y && gamma && beta, "%s: null pointer", what);
    if (int rc = check_rows(ctx, what, rows, C, x_stride, "x")) return rc;
    if (int rc = check_rows(ctx, what, rows, C, y_stride, "y")) return rc;
    if (int rc = check_alias(ctx, what, x, x_stride, "x", y, y_stride, "y", rows, C, dtype)) return rc;
    NormArgs a{x, x_stride, nullptr, 0, y, y_stride, gamma, beta, rows, static_cast<int>(C), 1, eps};
    return launch_norm(ctx, Norm::Layer, a, dtype, what);
}

int neko_hip_rmsnorm(neko_hip_ctx* ctx, const void* x, int64_t x_stride, void* y, int64_t y_stride, const float* w,
                     int64_t rows, int64_t C, float eps, int dtype) {
    const char* what = "neko_hip_rmsnorm";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && C > 0 && C <= 0x7fffffff, "%s: bad shape rows=%lld C=%lld", what, (long long)rows,
                 (long long)C);
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, x && y && w, "%s: null pointer", what);
    if (int rc = check_rows(ctx, what, rows, C, x_stride, "x")) return rc;
    if (int rc = check_rows(ctx, what, rows, C, y_stride, "y")) return rc;
    if (int rc = check_alias(ctx, what, x, x_stride, "x", y, y_stride, "y", rows, C, dtype)) return rc;
    NormArgs a{x, x_stride, nullptr, 0, y, y_stride, w, nullptr, rows, static_cast<int>(C), 1, eps};
    return launch_norm(ctx, Norm::Rms, a, dtype, what);
}

int neko_hip_add_rmsnorm(neko_hip_ctx* ctx, void* x, int64_t x_stride, const void* delta, int64_t delta_stride, void* xn,
                         int64_t xn_stride, const float* w, int64_t rows, int64_t C, float eps, int dtype) {
    const char* what = "neko_hip_add_rmsnorm";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && C > 0 && C <= 0x7fffffff, "%s: bad shape rows=%lld C=%lld", what, (long long)rows,
                 (long long)C);
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, x && delta && xn && w, "%s: null pointer", what);
    if (int rc = check_rows(ctx, what, rows, C, x_stride, "x")) return rc;
    if (int rc = check_rows(ctx, what, rows, C, delta_stride, "delta")) return rc;
    if (int rc = check_rows(ctx, what, rows, C, xn_stride, "xn")) return rc;
    if (int rc = check_alias(ctx, what, x, x_stride, "x", xn, xn_stride, "xn", rows, C, dtype, false)) return rc;
    if (int rc = check_alias(ctx, what, delta, delta_stride, "delta", xn, xn_stride, "xn", rows, C, dtype, false)) return rc;
    if (int rc = check_alias(ctx, what, delta, delta_stride, "delta", x, x_stride, "x", rows, C, dtype)) return rc;
    NormArgs a{x, x_stride, delta, delta_stride, xn, xn_stride, w, nullptr, rows, static_cast<int>(C), 1, eps};
    return launch_norm(ctx, Norm::AddRms, a, dtype, what);
}

int neko_hip_gated_rmsnorm(neko_hip_ctx* ctx, const void* y, int64_t y_stride, const void* z, int64_t z_stride, void* out,
                           int64_t out_stride, const float* w, int64_t rows, int64_t D, int groups, float eps, int dtype) {
    const char* what = "neko_hip_gated_rmsnorm";
    NEKO_ENTER(ctx);
    NEKO_REQUIRE(ctx, valid_dtype(dtype), "%s: bad dtype %d", what, dtype);
    NEKO_REQUIRE(ctx, rows >= 0 && D > 0 && D <= 0x7fffffff && groups > 0 && D % groups == 0,
                 "%s: bad shape rows=%lld D=%lld groups=%d", what, (long long)rows, (long long)D, groups);
    if (rows == 0) return NEKO_OK;
    NEKO_REQUIRE(ctx, y && z && out && w, "%s: null pointer", what);
    if (int rc = check_rows(ctx, what, rows, D, y_stride, "y")) return rc;
    if (int rc = check_rows(ctx, what, rows, D, z_stride, "z")) return rc;
    if (int rc = check_rows(ctx, what, rows, D, out_stride, "out")) return rc;
    if (int rc = check_alias(ctx, what, y, y_stride, "y", out, out_stride, "out", rows, D, dtype)) return rc;
    if (int rc = check_alias(ctx, what, z, z_stride, "z", out, out_stride, "out", rows, D, dtype, false)) return rc;
    NEKO_REQUIRE(ctx, rows <= INT64_MAX / groups, "%s: too many rows", what);
    NormArgs a{y, y_stride, z, z_stride, out, out_stride, w, nullptr, rows * groups, static_cast<int>(D / groups), groups, eps};
    return launch_norm(ctx, Norm::Gated, a, dtype, what);
}

}  // extern "C"
