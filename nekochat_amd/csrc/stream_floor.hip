// Streaming-floor kernels for measurement (libneko_floor.so, loaded by bench.py only; not part of the
// C ABI in include/neko_hip.h). They move bytes and do nothing else, so their times under the same
// events and cache flush as the layer ops give the practical floor an op of the same byte pattern can
// reach on this GPU: an empty kernel (launch and completion cost), a 16-byte-per-lane copy (read n,
// write n), a two-input stream (read 2n, write n: SwiGLU's byte counts), the same with SwiGLU's row
// layout (both inputs halves of one row), an in-place read-and-write-back of the first part of each
// row (the q/k RoPE's layout; flat, and in that kernel's per-wave token order), rows moved in the
// one-round row kernels' shape (every row of a wave loaded before any store), the embedding gather's
// pattern (table rows read through token ids, contiguous output rows written), the residual add +
// RMSNorm's, the KV store's, the fused q/k RoPE + KV store's and the gated norm's byte patterns, and a
// read-only sweep. The flat copies, SwiGLU's layout and the flat in-place rewrite also come with their
// workgroups' data in runs of X per XCD (xcd_block, device.h), the order the SwiGLU and q/k RoPE
// kernels use.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

__global__ void empty_kernel() {}

// Chunk i = (block * ITEMS + k) * 256 + thread: each load instruction of a wave covers 1 KB of
// contiguous bytes; all ITEMS loads are issued before the first store.
// Data block of workgroup b of G: b itself (X = 0) or in runs of X per XCD.
template <int X>
__device__ __forceinline__ uint32_t data_block(uint32_t b, uint32_t G) {
    if constexpr (X == 0) return b;
    else return neko_hip::xcd_block<X>(b, G);
}

template <int ITEMS, bool NTL, bool NTS, int X = 0>
__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst, int64_t n) {
    const int64_t base = static_cast<int64_t>(data_block<X>(blockIdx.x, gridDim.x)) * 256 * ITEMS + threadIdx.x;
    u32x4 v[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t i = base + k * 256;
        v[k] = i < n ? ld<NTL>(src + i) : u32x4{};
    }
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t i = base + k * 256;
        if (i < n) st<NTS>(dst + i, v[k]);
    }
}

// dst[i] = a[i] ^ b[i]: two read streams, one write stream.
template <bool NTL, bool NTS>
__global__ __launch_bounds__(256) void copy2_kernel(const u32x4* __restrict__ a, const u32x4* __restrict__ b,
                                                    u32x4* __restrict__ dst, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) st<NTS>(dst + i, ld<NTL>(a + i) ^ ld<NTL>(b + i));
}

// Reads every chunk; a lane stores only if its xor equals a value the data never produces in practice,
// which keeps the loads without writing.
template <int ITEMS>
__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ src, int64_t n, u32x4* sink) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * ITEMS + threadIdx.x;
    u32x4 acc{};
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t i = base + k * 256;
        if (i < n) acc ^= ld<true>(src + i);
    }
    if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u) sink[threadIdx.x] = acc;
}

// SwiGLU's layout without its arithmetic: rows of h hold two halves of `cpr` chunks; out[r][c] =
// h[r][c] ^ h[r][cpr + c], the flattened (row, chunk) index split with a division by cpr.
template <bool NTL, bool NTS, int X = 0>
__global__ __launch_bounds__(256) void rows2_kernel(const u32x4* __restrict__ h, int64_t hs, u32x4* __restrict__ out,
                                                    int64_t os, uint32_t cpr, uint32_t items) {
    const uint32_t idx = data_block<X>(blockIdx.x, gridDim.x) * 256u + threadIdx.x;
    if (idx >= items) return;
    const uint32_t row = idx / cpr, col = idx - row * cpr;
    const u32x4* hp = h + row * hs + col;
    st<NTS>(out + row * os + col, ld<NTL>(hp) ^ ld<NTL>(hp + cpr));
}

// The q/k RoPE's layout without its arithmetic: the first `cpr` chunks of each row (stride `stride`
// chunks) are read and written back in place, xored with `key` (0 at run time, unknown to the
// compiler, so every store is kept).
template <bool NTL, bool NTS, int X = 0>
__global__ __launch_bounds__(256) void inplace_kernel(u32x4* buf, int64_t stride, uint32_t cpr, uint32_t items, uint32_t key) {
    const uint32_t idx = data_block<X>(blockIdx.x, gridDim.x) * 256u + threadIdx.x;
    if (idx >= items) return;
    const uint32_t row = idx / cpr, col = idx - row * cpr;
    u32x4* p = buf + row * stride + col;
    st<NTS>(p, ld<NTL>(p) ^ key);
}

// The same bytes in the q/k RoPE kernel's schedule: wave w of nw rewrites rows w, w + nw, ... (the
// first 64 * CPL chunks of each, in place, xored with `key`), holding one row in registers and
// refilling each chunk with the wave's next row right after storing it; the last row is peeled so no
// load is under a branch.
template <int CPL, bool NTL, bool NTS>
__global__ __launch_bounds__(256) void inplace_rows_kernel(u32x4* buf, int64_t stride, int64_t rows, uint32_t key) {
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (t >= rows) return;
    u32x4 r[CPL];
    const u32x4* p0 = buf + t * stride + lane;
#pragma unroll
    for (int j = 0; j < CPL; j++) r[j] = ld<NTL>(p0 + 64 * j);
    for (; t + nw < rows; t += nw) {
        u32x4* q = buf + t * stride + lane;
        const u32x4* nx = buf + (t + nw) * stride + lane;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            st<NTS>(q + 64 * j, r[j] ^ key);
            r[j] = ld<NTL>(nx + 64 * j);
        }
    }
    u32x4* q = buf + t * stride + lane;
#pragma unroll
    for (int j = 0; j < CPL; j++) st<NTS>(q + 64 * j, r[j] ^ key);
}

// Rows moved in the shape of the one-round row kernels: wave w of nw takes rows w, w + nw, ...,
// (R of them, nw * R >= rows), issues every load of all R rows before its first store, then stores
// them; each row is CPL 16-byte chunks per lane (64 * CPL chunks), read at `src` and written at `dst`
// (the same pointer and stride for an in-place rewrite), xored with `key`. SYNC: a workgroup barrier
// between the loads and the stores (the workgroup's reads all land before any of its writes, as in
// the row kernels that stage their weights behind a barrier).
template <int R, int CPL, bool SYNC>
__global__ __launch_bounds__(256) void rows_up_kernel(const u32x4* src, int64_t ss, u32x4* dst, int64_t ds, int64_t rows,
                                                      uint32_t key) {
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    u32x4 v[R][CPL];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int64_t row = w + r * nw;
        const u32x4* p = src + (row < rows ? row : 0) * ss + lane;
#pragma unroll
        for (int j = 0; j < CPL; j++) v[r][j] = __builtin_nontemporal_load(p + 64 * j);
    }
    if constexpr (SYNC) __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int64_t row = w + r * nw;
        if (row >= rows) break;
        u32x4* p = dst + row * ds + lane;
#pragma unroll
        for (int j = 0; j < CPL; j++) __builtin_nontemporal_store(v[r][j] ^ key, p + 64 * j);
    }
}

// The embedding gather's byte pattern without its decode: wave w takes tokens TPW w .. TPW w + TPW - 1
// (their ids in one load), reads each token's table row (row_chunks 16-byte chunks, lane l chunks l,
// l + 64, ...) and writes out_chunks 16-byte chunks of output per token (lane l chunks l, l + 64, ...:
// 1 KB of contiguous output per store instruction), every output chunk the xor of the lane's row
// chunks with `key`. row_chunks <= 256, out_chunks <= 256. NTL: non-temporal row loads (plain ones keep
// the rows that repeated ids read again in L2).
template <int TPW, bool NTL>
__global__ __launch_bounds__(256) void gather_kernel(const int32_t* ids, int64_t T, const u32x4* table, int64_t row_stride,
                                                     int row_chunks, u32x4* out, int64_t out_stride, int out_chunks,
                                                     uint32_t key) {
    const int lane = threadIdx.x & 63;
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * TPW;
    if (t0 >= T) return;
    const int32_t my_id = lane < TPW && t0 + lane < T ? ids[t0 + lane] : 0;
    u32x4 acc[TPW];
#pragma unroll
    for (int k = 0; k < TPW; k++) {
        const int64_t id = __builtin_amdgcn_readlane(my_id, k);
        const u32x4* row = table + id * row_stride;
        acc[k] = u32x4{key, key, key, key};
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (64 * j + lane < row_chunks) acc[k] ^= NTL ? __builtin_nontemporal_load(row + 64 * j + lane) : row[64 * j + lane];
    }
#pragma unroll
    for (int k = 0; k < TPW; k++) {
        if (t0 + k >= T) break;
        u32x4* o = out + (t0 + k) * out_stride;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (64 * j + lane < out_chunks) o[64 * j + lane] = acc[k] ^ u32x4{static_cast<uint32_t>(j), 0u, 0u, 0u};
    }
}

// The residual add + RMSNorm's bytes: two streams in (a, b), two out (a rewritten in place, c): chunk
// i = (block * ITEMS + k) * 256 + thread as in copy_kernel.
template <int ITEMS, bool NTL, bool NTS>
__global__ __launch_bounds__(256) void add2_kernel(u32x4* a, const u32x4* __restrict__ b, u32x4* __restrict__ c, int64_t n,
                                                   uint32_t key) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * ITEMS * 256 + threadIdx.x;
    u32x4 va[ITEMS], vb[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t i = base + k * 256;
        if (i < n) {
            va[k] = ld<NTL>(a + i);
            vb[k] = ld<NTL>(b + i);
        }
    }
#pragma unroll
    for (int k = 0; k < ITEMS; k++) {
        const int64_t i = base + k * 256;
        if (i < n) {
            st<NTS>(a + i, va[k] ^ vb[k]);
            st<NTS>(c + i, va[k] ^ key);
        }
    }
}

// One workgroup per row (all three below): `row`-th rows of the buffers, 16-byte chunks j.
// The KV store's bytes: the k and v parts of each qkv row (2 * cw chunks, contiguous) read, the first
// cw chunks written to dst1's row, the next cw to dst2's.
__global__ __launch_bounds__(256) void split2_kernel(const u32x4* __restrict__ src, int64_t ss, int cw, u32x4* __restrict__ d1,
                                                     u32x4* __restrict__ d2, int64_t ds) {
    const int64_t row = blockIdx.x;
    for (int j = threadIdx.x; j < 2 * cw; j += 256) {
        const u32x4 v = ld<true>(src + row * ss + j);
        if (j < cw) d1[row * ds + j] = v;
        else d2[row * ds + j - cw] = v;
    }
}

// The q/k RoPE fused with the KV store: the first cq chunks of each row rewritten in place, the last
// ck of those also written to kd's row, and the cv chunks after them (v) copied to vd's row.
__global__ __launch_bounds__(256) void inplace_kv_kernel(u32x4* buf, int64_t stride, int cq, int ck, int cv,
                                                         u32x4* __restrict__ kd, u32x4* __restrict__ vd, int64_t ds,
                                                         uint32_t key) {
    const int64_t row = blockIdx.x;
    u32x4* r = buf + row * stride;
    for (int j = threadIdx.x; j < cq + cv; j += 256) {
        const u32x4 v = ld<true>(r + j);
        if (j < cq) {
            const u32x4 w = v ^ key;
            r[j] = w;
            if (j >= cq - ck) kd[row * ds + j - (cq - ck)] = w;
        } else {
            vd[row * ds + j - cq] = v;
        }
    }
}

// The gated norm's bytes: a y row and a z row (each its own buffer and stride) read, an output row
// written (o may be y: in place).
__global__ __launch_bounds__(256) void gate_kernel(const u32x4* y, int64_t ys, const u32x4* __restrict__ z, int64_t zs,
                                                   u32x4* o, int64_t os, int cw) {
    const int64_t row = blockIdx.x;
    for (int j = threadIdx.x; j < cw; j += 256) {
        const u32x4 a = ld<true>(y + row * ys + j), b = ld<true>(z + row * zs + j);
        o[row * os + j] = a ^ b;
    }
}

bool ok16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int ITEMS>
hipError_t launch_copy(const u32x4* s, u32x4* d, int64_t n, int ntl, int nts, hipStream_t st) {
    const int64_t blocks = (n + 256 * ITEMS - 1) / (256 * ITEMS);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>(blocks)), b(256);
    if (ntl && nts) hipLaunchKernelGGL((copy_kernel<ITEMS, true, true>), g, b, 0, st, s, d, n);
    else if (ntl) hipLaunchKernelGGL((copy_kernel<ITEMS, true, false>), g, b, 0, st, s, d, n);
    else if (nts) hipLaunchKernelGGL((copy_kernel<ITEMS, false, true>), g, b, 0, st, s, d, n);
    else hipLaunchKernelGGL((copy_kernel<ITEMS, false, false>), g, b, 0, st, s, d, n);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Empty kernel over `blocks` workgroups of 256 threads.
int neko_floor_empty(int blocks, void* stream) {
    if (blocks < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream));
    return hipGetLastError();
}

// dst[0, bytes) = src[0, bytes); bytes % 16 == 0, 16-byte aligned, disjoint. items: 16-byte chunks
// per lane (1, 2, 4 or 8); nt_load / nt_store: non-temporal loads / stores.
int neko_floor_copy(const void* src, void* dst, size_t bytes, int items, int nt_load, int nt_store, void* stream) {
    if (!ok16(src) || !ok16(dst) || bytes % 16) return hipErrorInvalidValue;
    const auto* s = static_cast<const u32x4*>(src);
    auto* d = static_cast<u32x4*>(dst);
    const int64_t n = static_cast<int64_t>(bytes / 16);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    switch (items) {
        case 1: return launch_copy<1>(s, d, n, nt_load, nt_store, st);
        case 2: return launch_copy<2>(s, d, n, nt_load, nt_store, st);
        case 4: return launch_copy<4>(s, d, n, nt_load, nt_store, st);
        case 8: return launch_copy<8>(s, d, n, nt_load, nt_store, st);
    }
    return hipErrorInvalidValue;
}

// dst[0, out_bytes) = a ^ b over the same range: reads 2 * out_bytes, writes out_bytes.
int neko_floor_copy2(const void* a, const void* b, void* dst, size_t out_bytes, int nt_load, int nt_store, void* stream) {
    if (!ok16(a) || !ok16(b) || !ok16(dst) || out_bytes % 16) return hipErrorInvalidValue;
    const int64_t n = static_cast<int64_t>(out_bytes / 16);
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>(blocks)), bl(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* pa = static_cast<const u32x4*>(a);
    const auto* pb = static_cast<const u32x4*>(b);
    auto* d = static_cast<u32x4*>(dst);
    if (nt_load && nt_store) hipLaunchKernelGGL((copy2_kernel<true, true>), g, bl, 0, st, pa, pb, d, n);
    else if (nt_load) hipLaunchKernelGGL((copy2_kernel<true, false>), g, bl, 0, st, pa, pb, d, n);
    else if (nt_store) hipLaunchKernelGGL((copy2_kernel<false, true>), g, bl, 0, st, pa, pb, d, n);
    else hipLaunchKernelGGL((copy2_kernel<false, false>), g, bl, 0, st, pa, pb, d, n);
    return hipGetLastError();
}

// out[r][0, half) = h[r][0, half) ^ h[r][half, 2 half) for rows of h_stride / out_stride bytes;
// half, the strides and the pointers multiples of 16 bytes; rows * half / 16 < 2^32.
int neko_floor_rows2(const void* h, int64_t h_stride, void* out, int64_t out_stride, int64_t rows, int64_t half, int nt_load,
                     int nt_store, void* stream) {
    if (!ok16(h) || !ok16(out) || half % 16 || h_stride % 16 || out_stride % 16 || half <= 0 || rows <= 0)
        return hipErrorInvalidValue;
    const int64_t cpr = half / 16, items = rows * cpr;
    if (items >= (int64_t(1) << 32) - 256) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>((items + 255) / 256)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* hp = static_cast<const u32x4*>(h);
    auto* op = static_cast<u32x4*>(out);
    const int64_t hs = h_stride / 16, os = out_stride / 16;
    const uint32_t c = static_cast<uint32_t>(cpr), n = static_cast<uint32_t>(items);
    if (nt_load && nt_store) hipLaunchKernelGGL((rows2_kernel<true, true>), g, b, 0, st, hp, hs, op, os, c, n);
    else if (nt_load) hipLaunchKernelGGL((rows2_kernel<true, false>), g, b, 0, st, hp, hs, op, os, c, n);
    else if (nt_store) hipLaunchKernelGGL((rows2_kernel<false, true>), g, b, 0, st, hp, hs, op, os, c, n);
    else hipLaunchKernelGGL((rows2_kernel<false, false>), g, b, 0, st, hp, hs, op, os, c, n);
    return hipGetLastError();
}

// buf[r][0, width) read and written back unchanged, in place, for rows of `stride` bytes; width,
// stride and buf multiples of 16 bytes; rows * width / 16 < 2^32.
int neko_floor_inplace(void* buf, int64_t stride, int64_t rows, int64_t width, int nt_load, int nt_store, void* stream) {
    if (!ok16(buf) || width % 16 || stride % 16 || width <= 0 || rows <= 0 || stride < width) return hipErrorInvalidValue;
    const int64_t cpr = width / 16, items = rows * cpr;
    if (items >= (int64_t(1) << 32) - 256) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>((items + 255) / 256)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    auto* p = static_cast<u32x4*>(buf);
    const int64_t s = stride / 16;
    const uint32_t c = static_cast<uint32_t>(cpr), n = static_cast<uint32_t>(items);
    if (nt_load && nt_store) hipLaunchKernelGGL((inplace_kernel<true, true>), g, b, 0, st, p, s, c, n, 0u);
    else if (nt_load) hipLaunchKernelGGL((inplace_kernel<true, false>), g, b, 0, st, p, s, c, n, 0u);
    else if (nt_store) hipLaunchKernelGGL((inplace_kernel<false, true>), g, b, 0, st, p, s, c, n, 0u);
    else hipLaunchKernelGGL((inplace_kernel<false, false>), g, b, 0, st, p, s, c, n, 0u);
    return hipGetLastError();
}

// buf[r][0, width) read and written back unchanged, in place, by `waves` waves in the q/k RoPE
// kernel's token order (wave w: rows w, w + waves', ... with waves' = waves rounded up to 4); width
// must be 10240 bytes (640 chunks: 32 + 8 heads of 128 halves), stride a multiple of 16 bytes.
int neko_floor_inplace_rows(void* buf, int64_t stride, int64_t rows, int64_t width, int waves, int nt_load, int nt_store,
                            void* stream) {
    constexpr int kCpl = 10;
    if (!ok16(buf) || width != 64 * 16 * kCpl || stride % 16 || stride < width || rows <= 0 || waves <= 0)
        return hipErrorInvalidValue;
    const int64_t w = waves < rows ? waves : rows;
    const dim3 g(static_cast<uint32_t>((w + 3) / 4)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    auto* p = static_cast<u32x4*>(buf);
    const int64_t s = stride / 16;
    if (nt_load && nt_store) hipLaunchKernelGGL((inplace_rows_kernel<kCpl, true, true>), g, b, 0, st, p, s, rows, 0u);
    else if (nt_load) hipLaunchKernelGGL((inplace_rows_kernel<kCpl, true, false>), g, b, 0, st, p, s, rows, 0u);
    else if (nt_store) hipLaunchKernelGGL((inplace_rows_kernel<kCpl, false, true>), g, b, 0, st, p, s, rows, 0u);
    else hipLaunchKernelGGL((inplace_rows_kernel<kCpl, false, false>), g, b, 0, st, p, s, rows, 0u);
    return hipGetLastError();
}

// `rows` rows of 64 * cpl 16-byte chunks copied from src (row stride s_stride bytes) to dst (d_stride)
// by ceil(rows / r) waves, each loading its r rows (rows w, w + nw, ...) before storing them (sync:
// with a workgroup barrier between); src == dst with equal strides rewrites in place. (r, cpl) in
// {1, 2, 3} x {5, 10}; strides multiples of 16.
int neko_floor_rows_up(const void* src, int64_t s_stride, void* dst, int64_t d_stride, int64_t rows, int r, int cpl,
                       int sync, void* stream) {
    if (!ok16(src) || !ok16(dst) || s_stride % 16 || d_stride % 16 || rows <= 0 || r < 1 || r > 3 ||
        (cpl != 5 && cpl != 10) || s_stride < 1024 * cpl || d_stride < 1024 * cpl)
        return hipErrorInvalidValue;
    const int64_t waves = (rows + r - 1) / r;
    const dim3 g(static_cast<uint32_t>((waves + 3) / 4)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* sp = static_cast<const u32x4*>(src);
    auto* dp = static_cast<u32x4*>(dst);
    const int64_t ss = s_stride / 16, dsd = d_stride / 16;
    // The grid holds ceil(waves / 4) * 4 waves; the kernel's nw is that count, so rows w + k nw with
    // k < r cover every row exactly once.
    const int64_t nw = static_cast<int64_t>(g.x) * 4;
    if (nw * r < rows) return hipErrorInvalidValue;
#define NEKO_ROWS_UP(R, C)                                                                                       \
    if (r == R && cpl == C) {                                                                                    \
        if (sync) hipLaunchKernelGGL((rows_up_kernel<R, C, true>), g, b, 0, st, sp, ss, dp, dsd, rows, 0u);       \
        else hipLaunchKernelGGL((rows_up_kernel<R, C, false>), g, b, 0, st, sp, ss, dp, dsd, rows, 0u);          \
    }
    NEKO_ROWS_UP(1, 5) NEKO_ROWS_UP(2, 5) NEKO_ROWS_UP(3, 5) NEKO_ROWS_UP(1, 10) NEKO_ROWS_UP(2, 10) NEKO_ROWS_UP(3, 10)
#undef NEKO_ROWS_UP
    return hipGetLastError();
}

// The gather's bytes: for t < T, reads table row ids[t] (row_bytes of it; rows row_stride bytes apart)
// and writes out_bytes at out + t * out_stride; ids must index the table (the caller checks), sizes
// multiples of 16 bytes up to 4 KB, tpw (tokens per wave) 1, 2 or 4, ntl: non-temporal row loads.
int neko_floor_gather(const int32_t* ids, int64_t T, const void* table, int64_t row_stride, int64_t row_bytes, void* out,
                      int64_t out_stride, int64_t out_bytes, int tpw, int ntl, void* stream) {
    if (!ok16(table) || !ok16(out) || row_stride % 16 || out_stride % 16 || row_bytes % 16 || out_bytes % 16 ||
        row_bytes <= 0 || row_bytes > 4096 || out_bytes <= 0 || out_bytes > 4096 || row_stride < row_bytes ||
        out_stride < out_bytes || T <= 0 || (tpw != 1 && tpw != 2 && tpw != 4))
        return hipErrorInvalidValue;
    const int64_t blocks = (T + 4 * tpw - 1) / (4 * tpw);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>(blocks)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* tp = static_cast<const u32x4*>(table);
    auto* op = static_cast<u32x4*>(out);
    const int rc = static_cast<int>(row_bytes / 16), oc = static_cast<int>(out_bytes / 16);
#define NEKO_FLOOR_GATHER(TPW, NTL) \
    hipLaunchKernelGGL((gather_kernel<TPW, NTL>), g, b, 0, st, ids, T, tp, row_stride / 16, rc, op, out_stride / 16, oc, 0u)
    if (tpw == 1 && ntl) NEKO_FLOOR_GATHER(1, true);
    else if (tpw == 1) NEKO_FLOOR_GATHER(1, false);
    else if (tpw == 2 && ntl) NEKO_FLOOR_GATHER(2, true);
    else if (tpw == 2) NEKO_FLOOR_GATHER(2, false);
    else if (ntl) NEKO_FLOOR_GATHER(4, true);
    else NEKO_FLOOR_GATHER(4, false);
#undef NEKO_FLOOR_GATHER
    return hipGetLastError();
}

// a[i] = a[i] ^ b[i], c[i] = a[i] ^ key over `bytes` of each (a in place; 1 or 4 chunks per lane).
int neko_floor_add2(void* a, const void* b, void* c, size_t bytes, int items, int nt_load, int nt_store, void* stream) {
    if (!ok16(a) || !ok16(b) || !ok16(c) || bytes % 16 || (items != 1 && items != 4)) return hipErrorInvalidValue;
    const int64_t n = static_cast<int64_t>(bytes / 16);
    const int64_t blocks = (n + 256 * items - 1) / (256 * items);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>(blocks)), bl(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    u32x4* pa = static_cast<u32x4*>(a);
    const u32x4* pb = static_cast<const u32x4*>(b);
    u32x4* pc = static_cast<u32x4*>(c);
#define NEKO_FLOOR_ADD2(I, L, S) hipLaunchKernelGGL((add2_kernel<I, L, S>), g, bl, 0, st, pa, pb, pc, n, 0u)
    if (items == 1 && nt_load && nt_store) NEKO_FLOOR_ADD2(1, true, true);
    else if (items == 1 && nt_load) NEKO_FLOOR_ADD2(1, true, false);
    else if (items == 1) NEKO_FLOOR_ADD2(1, false, false);
    else if (nt_load && nt_store) NEKO_FLOOR_ADD2(4, true, true);
    else if (nt_load) NEKO_FLOOR_ADD2(4, true, false);
    else NEKO_FLOOR_ADD2(4, false, false);
#undef NEKO_FLOOR_ADD2
    return hipGetLastError();
}

// For each of `rows` rows: 2 * width bytes at src + row * s_stride, the first width to dst1 + row *
// d_stride, the next width to dst2 + row * d_stride (strides in bytes, everything 16-byte aligned).
int neko_floor_split2(const void* src, int64_t s_stride, int64_t width, void* dst1, void* dst2, int64_t d_stride,
                      int64_t rows, void* stream) {
    if (!ok16(src) || !ok16(dst1) || !ok16(dst2) || s_stride % 16 || d_stride % 16 || width % 16 || width <= 0 ||
        rows <= 0 || rows > 0x7fffffff || s_stride < 2 * width || d_stride < width || width / 16 > (1 << 20))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(split2_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(src), s_stride / 16, static_cast<int>(width / 16), static_cast<u32x4*>(dst1),
                       static_cast<u32x4*>(dst2), d_stride / 16);
    return hipGetLastError();
}

// For each of `rows` rows of buf (stride bytes apart): its first qk_bytes rewritten in place, the last
// kv_bytes of those also written to kdst + row * d_stride, and the kv_bytes after them copied to vdst +
// row * d_stride.
int neko_floor_inplace_kv(void* buf, int64_t stride, int64_t rows, int64_t qk_bytes, int64_t kv_bytes, void* kdst,
                          void* vdst, int64_t d_stride, void* stream) {
    if (!ok16(buf) || !ok16(kdst) || !ok16(vdst) || stride % 16 || qk_bytes % 16 || kv_bytes % 16 || d_stride % 16 ||
        kv_bytes <= 0 || qk_bytes < kv_bytes || stride < qk_bytes + kv_bytes || d_stride < kv_bytes || rows <= 0 ||
        rows > 0x7fffffff || qk_bytes / 16 > (1 << 20))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(inplace_kv_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<u32x4*>(buf), stride / 16, static_cast<int>(qk_bytes / 16), static_cast<int>(kv_bytes / 16),
                       static_cast<int>(kv_bytes / 16), static_cast<u32x4*>(kdst), static_cast<u32x4*>(vdst), d_stride / 16, 0u);
    return hipGetLastError();
}

// For each of `rows` rows: width bytes of y and of z read (y_stride / z_stride bytes apart), width
// bytes written at out + row * out_stride (out may be y).
int neko_floor_gate(const void* y, int64_t y_stride, const void* z, int64_t z_stride, void* out, int64_t out_stride,
                    int64_t width, int64_t rows, void* stream) {
    if (!ok16(y) || !ok16(z) || !ok16(out) || y_stride % 16 || z_stride % 16 || out_stride % 16 || width % 16 ||
        width <= 0 || y_stride < width || z_stride < width || out_stride < width || rows <= 0 || rows > 0x7fffffff ||
        width / 16 > (1 << 20))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gate_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(y), y_stride / 16, static_cast<const u32x4*>(z), z_stride / 16,
                       static_cast<u32x4*>(out), out_stride / 16, static_cast<int>(width / 16));
    return hipGetLastError();
}

// The XCD-ordered forms, runs of `run` workgroups (64, 128 or 256) per XCD: neko_floor_copy with one
// chunk per lane, neko_floor_rows2 and neko_floor_inplace, same arguments otherwise.
int neko_floor_copy_x(const void* src, void* dst, size_t bytes, int nt_load, int nt_store, int run, void* stream) {
    if (!ok16(src) || !ok16(dst) || bytes % 16) return hipErrorInvalidValue;
    const int64_t n = static_cast<int64_t>(bytes / 16), blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff || nt_load != nt_store) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>(blocks)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* s = static_cast<const u32x4*>(src);
    auto* d = static_cast<u32x4*>(dst);
    const bool nt = nt_load != 0;
    switch (run * 2 + (nt ? 1 : 0)) {
        case 128: hipLaunchKernelGGL((copy_kernel<1, false, false, 64>), g, b, 0, st, s, d, n); break;
        case 129: hipLaunchKernelGGL((copy_kernel<1, true, true, 64>), g, b, 0, st, s, d, n); break;
        case 256: hipLaunchKernelGGL((copy_kernel<1, false, false, 128>), g, b, 0, st, s, d, n); break;
        case 257: hipLaunchKernelGGL((copy_kernel<1, true, true, 128>), g, b, 0, st, s, d, n); break;
        case 512: hipLaunchKernelGGL((copy_kernel<1, false, false, 256>), g, b, 0, st, s, d, n); break;
        case 513: hipLaunchKernelGGL((copy_kernel<1, true, true, 256>), g, b, 0, st, s, d, n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// SwiGLU's layout, non-temporal loads and plain stores (its own cache policy), XCD-ordered.
int neko_floor_rows2_x(const void* h, int64_t h_stride, void* out, int64_t out_stride, int64_t rows, int64_t half, int run,
                       void* stream) {
    if (!ok16(h) || !ok16(out) || half % 16 || h_stride % 16 || out_stride % 16 || half <= 0 || rows <= 0)
        return hipErrorInvalidValue;
    const int64_t cpr = half / 16, items = rows * cpr;
    if (items >= (int64_t(1) << 32) - 256) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>((items + 255) / 256)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* hp = static_cast<const u32x4*>(h);
    auto* op = static_cast<u32x4*>(out);
    const int64_t hs = h_stride / 16, os = out_stride / 16;
    const uint32_t c = static_cast<uint32_t>(cpr), n = static_cast<uint32_t>(items);
    switch (run) {
        case 64: hipLaunchKernelGGL((rows2_kernel<true, false, 64>), g, b, 0, st, hp, hs, op, os, c, n); break;
        case 128: hipLaunchKernelGGL((rows2_kernel<true, false, 128>), g, b, 0, st, hp, hs, op, os, c, n); break;
        case 256: hipLaunchKernelGGL((rows2_kernel<true, false, 256>), g, b, 0, st, hp, hs, op, os, c, n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// The flat in-place rewrite, plain loads and stores, XCD-ordered.
int neko_floor_inplace_x(void* buf, int64_t stride, int64_t rows, int64_t width, int run, void* stream) {
    if (!ok16(buf) || width % 16 || stride % 16 || width <= 0 || rows <= 0 || stride < width) return hipErrorInvalidValue;
    const int64_t cpr = width / 16, items = rows * cpr;
    if (items >= (int64_t(1) << 32) - 256) return hipErrorInvalidValue;
    const dim3 g(static_cast<uint32_t>((items + 255) / 256)), b(256);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    auto* p = static_cast<u32x4*>(buf);
    const int64_t s = stride / 16;
    const uint32_t c = static_cast<uint32_t>(cpr), n = static_cast<uint32_t>(items);
    switch (run) {
        case 64: hipLaunchKernelGGL((inplace_kernel<false, false, 64>), g, b, 0, st, p, s, c, n, 0u); break;
        case 128: hipLaunchKernelGGL((inplace_kernel<false, false, 128>), g, b, 0, st, p, s, c, n, 0u); break;
        case 256: hipLaunchKernelGGL((inplace_kernel<false, false, 256>), g, b, 0, st, p, s, c, n, 0u); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Reads src[0, bytes) (non-temporal, 4 chunks per lane); sink: 4 KB of device memory (256 chunks).
int neko_floor_read(const void* src, size_t bytes, void* sink, void* stream) {
    if (!ok16(src) || !ok16(sink) || bytes % 16) return hipErrorInvalidValue;
    const int64_t n = static_cast<int64_t>(bytes / 16);
    const int64_t blocks = (n + 1023) / 1024;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((read_kernel<4>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(src), n, static_cast<u32x4*>(sink));
    return hipGetLastError();
}

}  // extern "C"
