/*
 * neko_hip: MI355X (gfx950) kernels for NekoChat's per-row transformer layer ops, behind a C ABI.
 *
 * Reference interfaces replaced (paths relative to the reference's app/architecture/shared/cpp/):
 *   - the GPU backend contract neko::gpu::ComputeBackend (gpu/compute.h:24-45): buffers, upload /
 *     download, ordered dispatch, submitAndWait -- the HIP adapter (nekochat_amd/csrc/hip_backend.cpp)
 *     implements it over the functions below;
 *   - its per-kernel dispatches Embed / LayerNorm / Rope / SiluMul (gpu/compute.h:17, shaders
 *     embed.comp, layernorm.comp, rope.comp, silu_mul.comp), plus the CPU-only Granite gated norm
 *     (granite/cpp/granite_model.cpp:278-287) and standalone GELU (cpu_ops.cpp:20-23);
 *   - the host codecs quantRowBytes / quantizeMatrix (quant.h:32,57) and Qwen3Model::ropeTable
 *     (qwen3/cpp/qwen3_model.cpp:102-114).
 *
 * Conventions
 *   - Every function returns an int status: NEKO_OK (0) or a negative NEKO_ERR_*; nothing throws.
 *     The message of the last failure on a context is neko_hip_last_error(ctx).
 *   - One context per host thread. A context issues all work to one in-order HIP stream -- the
 *     device's null stream unless neko_hip_set_stream routes it elsewhere -- so every op is ordered
 *     after the previous one (the reference's "each dispatch is ordered after the previous",
 *     gpu/compute.h:38) without barriers. Ops only enqueue work; neko_hip_download and
 *     neko_hip_synchronize wait.
 *   - Device pointers are plain addresses from neko_hip_alloc (or any HIP allocation on the
 *     context's device). Sizes and strides are int64 element counts unless the name says bytes.
 *   - dtype selects the activation type: NEKO_DT_F16 (IEEE half, fp32 arithmetic inside, one RNE
 *     rounding per output) or NEKO_DT_F32 (the reference's own activation type). Norm and gate
 *     weights (gamma, beta, w, wqk) are f32 arrays, as the reference keeps them.
 *   - Arithmetic follows the reference's CPU ops (cpu_ops.cpp:20-23,483-533): norms accumulate in
 *     double and round the scale to float; products are evaluated in the same order, unfused.
 */
#ifndef NEKO_HIP_H
#define NEKO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NEKO_OK 0
#define NEKO_ERR_INVALID (-1)     /* bad argument: null pointer, size, stride, alignment or format */
#define NEKO_ERR_HIP (-2)         /* a HIP runtime call or kernel launch failed */
#define NEKO_ERR_NO_DEVICE (-3)   /* no usable gfx950 device */
#define NEKO_ERR_UNSUPPORTED (-4) /* valid request this library does not implement */

typedef enum { NEKO_DT_F32 = 0, NEKO_DT_F16 = 1 } neko_dtype;

/* Weight row formats, numbered as the reference's WeightFormat (quant.h:19). */
typedef enum { NEKO_FMT_F16 = 0, NEKO_FMT_FP8 = 1, NEKO_FMT_FP4 = 2 } neko_weight_format;

typedef struct neko_hip_ctx neko_hip_ctx;

/* ---------------------------------------------------------------- context and memory
 * Replace the ComputeBackend factory / create / upload / download / submitAndWait
 * (gpu/compute.h:28-44, vk_compute.cpp:459-466). */

/* Opens device `device`. *out is NULL on failure; the message of a failed create is available as
 * neko_hip_last_error(NULL). */
int neko_hip_create(int device, neko_hip_ctx** out);
/* Waits for outstanding work and releases any memory still allocated through the ctx. */
int neko_hip_destroy(neko_hip_ctx* ctx);
/* Last error message on ctx (or of the last failed neko_hip_create when ctx is NULL). Never NULL. */
const char* neko_hip_last_error(const neko_hip_ctx* ctx);
/* Device name and the largest single allocation (ComputeBackend::deviceName / maxBufferBytes). */
int neko_hip_device_name(neko_hip_ctx* ctx, char* buf, size_t buf_bytes);
size_t neko_hip_max_buffer_bytes(const neko_hip_ctx* ctx);
/* Routes subsequent work to a hipStream_t on the same device (e.g. a framework's current stream);
 * NULL selects the device's null stream, the default. The caller keeps ownership of the stream.
 * On a change the new stream is first made to wait (on the device) for the work already issued on
 * the previous one, so the context's ops stay ordered across the switch -- except when either stream
 * is under graph capture, where the caller orders the graph's launches. */
int neko_hip_set_stream(neko_hip_ctx* ctx, void* hip_stream);
void* neko_hip_get_stream(const neko_hip_ctx* ctx);

int neko_hip_alloc(neko_hip_ctx* ctx, size_t bytes, void** dev_ptr);
int neko_hip_free(neko_hip_ctx* ctx, void* dev_ptr);
/* Ordered on the context's stream; upload returns once src may be reused. */
int neko_hip_upload(neko_hip_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
/* Waits for all work queued before it, then copies. */
int neko_hip_download(neko_hip_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
int neko_hip_memset(neko_hip_ctx* ctx, void* dst_dev, int value, size_t bytes);
int neko_hip_synchronize(neko_hip_ctx* ctx);

/* ---------------------------------------------------------------- row norms */

/* LayerNorm over rows of C: y = (x - mean) * rstd * gamma + beta, two-pass mean / variance in
 * double (cpu_ops.cpp:483-500; GPU form layernorm.comp flags = 0). x and y are either the same rows
 * (same pointer and stride: in place) or disjoint; any other overlap is rejected (NEKO_ERR_INVALID). */
int neko_hip_layernorm(neko_hip_ctx* ctx, const void* x, int64_t x_stride, void* y, int64_t y_stride,
                       const float* gamma, const float* beta, int64_t rows, int64_t C, float eps, int dtype);

/* RMSNorm over rows of C: y = x * float(1/sqrt(sum(x^2)/C + eps)) * w (cpu_ops.cpp:502-511; GPU form
 * layernorm.comp flags = 1). x and y are the same rows (same pointer and stride: in place, which
 * cpu_ops.h:27 allows) or disjoint; other overlaps are rejected. Also the Qwen3 q/k head norm when
 * called on heads as rows (qwen3_model.cpp:250-251). */
int neko_hip_rmsnorm(neko_hip_ctx* ctx, const void* x, int64_t x_stride, void* y, int64_t y_stride, const float* w,
                     int64_t rows, int64_t C, float eps, int dtype);

/* Granite-4.0-H Mamba2 output gate + group RMSNorm: g = y * silu(z), then RMSNorm of each group of
 * D/groups channels with its slice of w, written to out (granite_model.cpp:278-287, which gates and
 * norms y in place). out is either y itself (same pointer and stride) or disjoint from it, and never
 * overlaps z. z rows have stride z_stride (the gate columns of the in_proj row,
 * granite_model.h:86-88). D % groups == 0. */
int neko_hip_gated_rmsnorm(neko_hip_ctx* ctx, const void* y, int64_t y_stride, const void* z, int64_t z_stride,
                           void* out, int64_t out_stride, const float* w, int64_t rows, int64_t D, int groups,
                           float eps, int dtype);

/* ---------------------------------------------------------------- attention prologue */

/* Qwen3 per-head q/k RMSNorm then NeoX half-split RoPE, in place on the q and k heads of each qkv
 * row (row = [q n_q*hd | k n_kv*hd | v n_kv*hd], stride row_stride); v is neither read nor written
 * (rope.comp:1-55, dispatch qwen3_model.cpp:313; CPU qwen3_model.cpp:249-253).
 *   wqk       f32 [2*hd]: q_norm weights then k_norm weights; NULL = rotation only (rope.comp flags 0).
 *   cs        f32 [n_pos][hd]: hd/2 (cos, sin) pairs per position (Qwen3Model::ropeTable layout).
 *   positions int32 [rows] per-row positions, or NULL for pos0 + row (the reference's GPU ABI).
 * Rows whose position lies outside [0, n_pos) are left untouched. hd even, hd <= 512. */
int neko_hip_qk_norm_rope(neko_hip_ctx* ctx, void* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                          int64_t pos0, const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos,
                          float eps, int dtype);

/* The same, fused with the KV-cache store that follows it (qwen3_model.cpp:249-256: rope, then
 * cpu::storeKv, cpu_ops.cpp:535-542; GPU kv_store.comp): after the q/k heads of a row are normed and
 * rotated, its rotated k heads and its v heads are also written as f16 to cache row = the row's
 * position, k_cache / v_cache being [cache_rows][n_kv*hd] halves. f16 activations are stored bit for
 * bit; f32 activations are rounded to f16 (RNE). Rows outside [0, n_pos) are untouched and store
 * nothing; cache_rows >= n_pos. Rows that share a position write the same cache row (which one lands
 * last is unspecified). */
int neko_hip_qk_norm_rope_kv(neko_hip_ctx* ctx, void* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                             int64_t pos0, const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos,
                             float eps, uint16_t* k_cache, uint16_t* v_cache, int64_t cache_rows, int dtype);

/* KV-cache store alone (cpu_ops.cpp:535-542; the GPU kernel KvStore, kv_store.comp:1-21): for each
 * row t, the width k values at qkv[t*row_stride + k_off] and v values at [... + v_off] are written as
 * f16 (RNE from f32; bit copies from f16) to k_cache / v_cache row positions[t] (or pos0 + t), rows of
 * width halves. Rows whose cache row is outside [0, cache_rows) are skipped. */
int neko_hip_store_kv(neko_hip_ctx* ctx, const void* qkv, int64_t row_stride, int64_t k_off, int64_t v_off, int64_t rows,
                      int64_t width, int64_t pos0, const int32_t* positions, uint16_t* k_cache, uint16_t* v_cache,
                      int64_t cache_rows, int dtype);

/* Causal grouped-query attention over the f16 KV caches (cpu::attention, cpu_ops.cpp:544-575; the GPU
 * kernel Attention, attention.comp, dispatched by qwen3_model.cpp:317 and gpt2_model.cpp:255): for
 * token t = 0 .. T-1 at position pos0 + t and query head h < n_head,
 *   out[t*out_stride + h*hd + d] = sum_j w_j v_j[d] / sum_j w_j,  w_j = exp(scale * q . k_j - max),
 * over cache rows j = 0 .. pos0 + t, where q = q[t*q_stride + h*hd ..] (dtype) and k_j / v_j are the hd
 * halves of k_cache / v_cache at j*n_kv*hd + (h / (n_head / n_kv))*hd (the reference's cache layout:
 * rows of n_kv*hd halves, holding positions 0 .. pos0 + T - 1). n_head a multiple of n_kv; hd even,
 * 2..256; the reference's scale is 1/sqrt(hd); caches 4-byte aligned. out may not overlap q or the
 * caches. f32 sums in another order than the reference's CPU loop (whose order its own shader does not
 * follow either): within 1e-6 relative of it at the tested shapes. */
int neko_hip_attention(neko_hip_ctx* ctx, const void* q, int64_t q_stride, const uint16_t* k_cache, const uint16_t* v_cache,
                       void* out, int64_t out_stride, int64_t T, int n_head, int n_kv, int hd, int64_t pos0, float scale,
                       int dtype);

/* ---------------------------------------------------------------- residual */

/* Residual add + RMSNorm: x[t] = x[t] + delta[t] (float add, rounded once to the activation type,
 * written back to x), then xn[t] = RMSNorm(x[t]) with weights w -- the reference's matmul epilogue
 * with kAccumulate (cpu_ops.cpp:123, dst = dst + v) followed by the next op's cpu::rmsNorm
 * (qwen3_model.cpp:264, cpu_ops.cpp:502-511), with the add moved out of the GEMM so the residual row
 * is read once for both. xn may not overlap x or delta; delta is either x itself (same pointer and
 * stride) or disjoint from it. */
int neko_hip_add_rmsnorm(neko_hip_ctx* ctx, void* x, int64_t x_stride, const void* delta, int64_t delta_stride, void* xn,
                         int64_t xn_stride, const float* w, int64_t rows, int64_t C, float eps, int dtype);

/* ---------------------------------------------------------------- activations */

/* SwiGLU: out[t][i] = gate / (1 + exp(-gate)) * up with gate = h[t][i], up = h[t][I + i]
 * (cpu_ops.cpp:526-533, silu_mul.comp). h rows hold gate then up (stride h_stride >= 2*I). out is
 * disjoint from h, or overwrites its gate halves (out == h, out_stride == h_stride). */
int neko_hip_swiglu(neko_hip_ctx* ctx, const void* h, int64_t h_stride, void* out, int64_t out_stride, int64_t rows,
                    int64_t I, int dtype);

/* GELU, tanh form: y = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))) over n contiguous elements
 * (cpu_ops.cpp:20-23; the matmul epilogue of matmul.comp:16-19). x and y are the same array or
 * disjoint. */
int neko_hip_gelu_tanh(neko_hip_ctx* ctx, const void* x, void* y, int64_t n, int dtype);

/* ---------------------------------------------------------------- embedding gather */

/* out[t] = dequant(table[tokens[t] - row_base]) (+ f32(wpe[pos0 + t])) for tokens with
 * row_base <= tokens[t] < row_base + rows; other tokens leave out[t] untouched, so a table split
 * into row chunks is gathered with one call per chunk (embed.comp:1-51, quant.cpp:230-253,
 * gpt2_model.cpp:182-187, qwen3_model.cpp:301-305).
 *   table     rows of row_bytes bytes in weight format fmt (quant.h:30-36 layout); row_bytes must
 *             be even and at least neko_quant_row_bytes(fmt, C). FP8/FP4 need C % 32 == 0.
 *   wpe       f16 [wpe_rows][C] position table added in f32, or NULL. Requires pos0 + T <= wpe_rows.
 *   out       rows of out_stride elements of out_dtype; f16 output is one RNE rounding of the f32
 *             result. Dequantisation is exact, so the output is bit-exact with the reference. */
int neko_hip_embed(neko_hip_ctx* ctx, const int32_t* tokens, int64_t T, const void* table, int64_t row_bytes, int fmt,
                   int64_t C, int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t wpe_rows, int64_t pos0,
                   void* out, int64_t out_stride, int out_dtype);

/* Granite's gather (granite_model.cpp:298-301): as neko_hip_embed without a position table, each
 * dequantised value then multiplied by `scale` in f32 (the model's embedding_multiplier: one f32
 * rounding, as the reference's x[c] *= embeddingMult), f16 output one RNE rounding of that. */
int neko_hip_embed_scaled(neko_hip_ctx* ctx, const int32_t* tokens, int64_t T, const void* table, int64_t row_bytes,
                          int fmt, int64_t C, int64_t row_base, int64_t rows, float scale, void* out, int64_t out_stride,
                          int out_dtype);

/* Load-time quantiser on the device (quantizeMatrix, quant.cpp:255-279, portable branch): rows x cols
 * weights (src_dtype f32, or f16 widened exactly; row stride src_stride elements, device memory)
 * encoded into device rows of neko_quant_row_bytes(*fmt_used, cols) bytes, bit-identical to
 * neko_quantize_rows and the reference (FP8 block scale and RNE codes, FP4 scale search with its
 * two least-squares refits, padding zeroed). cols % 32 != 0 stores F16, like the reference; FP8/FP4
 * need 16-byte aligned source rows and output. */
int neko_hip_quantize_rows(neko_hip_ctx* ctx, int fmt, int64_t rows, int64_t cols, const void* src, int64_t src_stride,
                           int src_dtype, uint8_t* dst, int* fmt_used);

/* ---------------------------------------------------------------- weight matmul */

/* y[t][n] (+)= act(x[t] . W[n] + bias[n]) for t < T, n < N: the reference's weight matmul,
 * cpu::matmul (cpu_ops.cpp:474-490, with matmulF16 :108-127 and matmulGeneric :455-472) and its GPU
 * kernels Matmul / MatmulQ8 / MatmulQ4 (gpu/compute.h:17; matmul.comp, matmul_q8.comp,
 * matmul_q4.comp), whose flags this keeps: NEKO_MM_GELU applies the GELU tanh form to the biased
 * sum, NEKO_MM_ACCUMULATE adds the result into y (dst = dst + v) instead of storing it.
 *   x      T rows of K activations (x_stride elements apart) of x_dtype.
 *   w      N weight rows of row_bytes bytes in format fmt (quant.h:30-36 layout, as written by
 *          neko_quantize_rows / neko_hip_quantize_rows); FP8/FP4 need K % 32 == 0.
 *   bias   f32 [N] or NULL.
 *   y      T rows of y_stride elements of y_dtype; may not overlap x or w. Column offsets (the
 *          shaders' nOffset) are a pointer offset into y.
 * The dot products are summed in f32 (f16 activations and weight codes exactly, each 32-block scaled
 * by its f16 scale) in a different order from the reference's sequential loop: results agree to f32
 * rounding of the sum. Fastest with f16 activations, 16-byte aligned x rows and weight rows (the
 * MFMA kernels). f32 activations with aligned rows: up to 8 tokens (16 for weights of at most
 * 2^24 elements) a VALU kernel (1.0-1.3x the f16 time at one token); beyond, each row split into
 * two f16 planes (scaled by a power of two) for the MFMA kernels, about 2-3x the f16 time, with the call's context workspace holding the
 * planes and sums. Other shapes take a generic kernel.
 * Shapes that split K keep f32 partial sums in a per-context workspace: allocated (or grown, to the
 * next power of two) by the first call that needs more; outgrown buffers are kept too (graphs
 * captured earlier still point at them), all until neko_hip_destroy -- together always less than the
 * live buffer. A call that would grow it while the context's stream is under
 * graph capture fails with NEKO_ERR_INVALID: make one uncaptured call at the largest shape first, or
 * capture neko_hip_matmul_noalloc. */
#define NEKO_MM_GELU 1
#define NEKO_MM_ACCUMULATE 2
int neko_hip_matmul(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w,
                    int64_t row_bytes, int fmt, int64_t N, const float* bias, void* y, int64_t y_stride, int flags,
                    int x_dtype, int y_dtype);

/* F16 weight rows with f16 activations from 512 tokens (64 for 16384 rows or more), without NEKO_MM_GELU and without a bias
 * added to an accumulated y (16-byte aligned y rows), on a stream not under graph capture:
 * neko_hip_matmul runs the product on hipBLASLt (the vendor GEMM library; measured faster than this library's own MFMA
 * kernels at prefill sizes), which draws up to 64 MiB of the context's workspace. enable = 0 keeps
 * every product of this context on the library's own kernels (enable = 1, the default, allows it).
 * No counterpart in the reference (its matmul is its own). */
int neko_hip_set_matmul_library(neko_hip_ctx* ctx, int enable);

/* neko_hip_matmul without any allocation: the same kernels, the same split of K and bit-identical
 * results (except for the F16 products neko_hip_matmul hands to hipBLASLt, which this entry point runs
 * on the library's own kernels, as neko_hip_matmul does with neko_hip_set_matmul_library(ctx, 0): the
 * same f32 sums in another order, within the same bound), but the memory neko_hip_matmul takes from
 * the context's workspace -- split-K partial sums,
 * and for f32 activations from 9 tokens (17 for weights of at most 2^24 elements) the two f16 planes
 * and their sums -- comes from a fixed 32 MiB array in device memory (one per GPU, held from the
 * library's first use on that GPU until the process ends). No counterpart in the reference: this is
 * for callers that cannot allocate -- code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc. A shape that needs more than the array holds (none of the Qwen3-0.6B/4B layer
 * projections with f16 activations at any token count; an FP8/FP4 vocabulary-sized product at 13-47
 * tokens, or f32 activations at prefill sizes, do) returns NEKO_ERR_UNSUPPORTED before anything is
 * launched. The array belongs to the first context that calls this entry point on its GPU until that
 * context is destroyed; a call through any other context returns NEKO_ERR_UNSUPPORTED. Calls through
 * the owning context are ordered on its stream; a caller that replays graphs captured from them on
 * several streams at once must order those replays itself. */
int neko_hip_matmul_noalloc(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w,
                            int64_t row_bytes, int fmt, int64_t N, const float* bias, void* y, int64_t y_stride,
                            int flags, int x_dtype, int y_dtype);

/* ---------------------------------------------------------------- host-side codecs */

/* Bytes per stored row (quant.cpp:199-208): F16 2*cols; FP8 / FP4 the codes (cols or cols/2
 * bytes) followed by cols/32 f16 block scales, zero-padded to a multiple of 16 bytes. */
size_t neko_quant_row_bytes(int fmt, int64_t cols);

/* Encodes rows x cols f32 weights (host memory) into rows of neko_quant_row_bytes(fmt, cols) bytes,
 * bit-identical to the reference's quantizeMatrix (quant.cpp:255-279, portable branch). cols % 32
 * != 0 stores F16, like the reference; *fmt_used reports the format written (may be NULL).
 * threads <= 0 uses every hardware thread. */
int neko_quantize_rows(int fmt, int64_t rows, int64_t cols, const float* src, uint8_t* dst, int threads,
                       int* fmt_used);

/* RoPE table (host memory): cs[p][2i] = float(cos(p * theta^(-2i/hd))), cs[p][2i+1] = float(sin(..))
 * for p < n_pos, i < hd/2, evaluated in double (qwen3_model.cpp:102-114). */
int neko_rope_table(double theta, int hd, int64_t n_pos, float* cs);

#ifdef __cplusplus
}
#endif

#endif /* NEKO_HIP_H */
