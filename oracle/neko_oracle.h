/*
 * CPU oracle for the fused layer ops: a plain-C restatement of the reference's own arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (nekochat_amd/, include/) links, loads or calls
 * this code. It is used by tests/ and by __graft_entry__.smoke() (for the expected results) and
 * by bench.py's cpu_baseline leg (as the timed CPU path). The GPU path never routes through it.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference's
 * app/architecture/). Activations in the reference are f32; the *_f16 entry points define the fp16
 * I/O semantics as: widen each input half exactly (common.h:33-55), run the reference op in f32
 * with its double accumulators, and round each output once to f16 with round-to-nearest-even
 * (common.h:57-80).
 *
 * How each function is pinned (checks live in tests/test_oracle.py):
 *   - f16 helpers: exhaustive over all 65536 halves (closed form and numpy's IEEE conversion);
 *     f32->f16 against numpy on special, boundary and random values.
 *   - layernorm / rmsnorm / gated rmsnorm / rope / silu_mul / gelu / rope table: bit-exact against
 *     the compiled reference (oracle/_ref, built from the reference sources) and the committed
 *     golden fixtures; plus long-double textbook forms within tolerance, constant/zero rows,
 *     pos 0 = identity and pair-norm preservation.
 *   - gated rmsnorm: the reference's gate (granite_model.cpp:21,282) does not compile on x86
 *     (unconditional <arm_neon.h>); it is pinned through the same restated gate composed with the
 *     compiled reference rmsNorm, plus a long-double textbook form.
 *   - FP8/FP4 codecs and row layout: exhaustive code tables (all 256 / 16 codes, with the special
 *     cases 0x7F/0xFF = +-480, 0x80 = -0, FP4 8 = -0), quantRowBytes closed form, and bit-exact
 *     encoder output against the compiled reference quantizeMatrix.
 *   - libm boundary (expf, tanhf, cos, sin, pow, sqrt): calls the C library exactly where the
 *     reference calls it; results at the last f32 ulp depend on the libm ("parity unpinned" at that
 *     level only; glibc here, bionic on the reference's phones).
 */
#ifndef NEKO_ORACLE_H
#define NEKO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 / bf16 scalar helpers (common.h:33-87) ---- */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
float oracle_bf16_to_f32(uint16_t b);
void oracle_f16_to_f32_n(const uint16_t* h, float* f, int64_t n);
void oracle_f32_to_f16_n(const float* f, uint16_t* h, int64_t n);

/* ---- f32 ops, the reference's exact arithmetic ---- */
float oracle_gelu(float x);                                                         /* cpu_ops.cpp:20-23 */
void oracle_layernorm(const float* x, float* y, const float* g, const float* b, int rows, int C,
                      float eps);                                                   /* cpu_ops.cpp:483-500 */
void oracle_rmsnorm(const float* x, float* y, const float* w, int rows, int C, float eps); /* :502-511 */
void oracle_rope(float* x, int n_heads, int hd, const float* cs);                  /* cpu_ops.cpp:513-524 */
void oracle_silu_mul(const float* h, float* out, int rows, int I);                 /* cpu_ops.cpp:526-533 */
float oracle_silu(float v);                                                         /* granite_model.cpp:21 */
/* In place on y (rows of D floats): y *= silu(z) then RMSNorm per group of D/groups channels
 * (granite_model.cpp:278-287). z rows have stride z_stride floats. */
void oracle_gated_rmsnorm(float* y, const float* z, int64_t z_stride, const float* w, int rows, int D,
                          int groups, float eps);
/* cs[p][i] = (cos(p * theta^(-2i/hd)), sin(...)) for p < n_pos, i < hd/2; row stride hd floats
 * (qwen3_model.cpp:102-114). */
void oracle_rope_table(double theta, int hd, int n_pos, float* cs);
/* KV-cache store (cpu_ops.cpp:535-542): k/v rows of width floats (stride src_stride) rounded to f16
 * into cache rows pos0 + t. */
void oracle_store_kv(const float* k, const float* v, int64_t src_stride, uint16_t* kc, uint16_t* vc, int width,
                     int64_t T, int64_t pos0);
/* Causal grouped-query attention over f16 caches (cpu_ops.cpp:544-575); out rows of n_head*hd floats. */
void oracle_attention(const float* q, int64_t q_stride, const uint16_t* kc, const uint16_t* vc, float* out, int64_t T,
                      int n_head, int n_kv, int hd, int64_t pos0);
/* Residual add (matmul kAccumulate epilogue, cpu_ops.cpp:123: x = x + d in float), then RMSNorm of
 * the updated rows into xn (qwen3_model.cpp:264, cpu_ops.cpp:502-511). x is updated in place. */
void oracle_add_rmsnorm(float* x, const float* d, float* xn, const float* w, int rows, int C, float eps);

/* ---- weight row formats (quant.h:19-58, quant.cpp) ---- */
enum { ORACLE_FMT_F16 = 0, ORACLE_FMT_FP8 = 1, ORACLE_FMT_FP4 = 2 };
size_t oracle_quant_row_bytes(int fmt, int cols);                                   /* quant.cpp:199-208 */
float oracle_decode_fp8(uint8_t c);                                                 /* quant.cpp:51-53 */
float oracle_decode_fp4(uint8_t c);                                                 /* quant.cpp:63-65 */
uint8_t oracle_encode_fp8(float y);                                                 /* quant.cpp:43-49 */
uint8_t oracle_encode_fp4(float y);                                                 /* quant.cpp:57-61 */
uint16_t oracle_fp4_block_scale(const float* xb);                                   /* quant.cpp:142-165 */
/* Encodes rows x cols floats into rows of oracle_quant_row_bytes(fmt, cols) bytes (padding zeroed).
 * cols % 32 != 0 falls back to F16 like quantizeMatrix (quant.cpp:255-279); returns the format used. */
int oracle_quantize_rows(int fmt, int64_t rows, int cols, const float* src, uint8_t* dst);
void oracle_dequantize_row(int fmt, int cols, const uint8_t* row, float* out);      /* quant.cpp:230-253 */

/* ---- fp16 I/O compositions (widen -> reference op -> RNE narrow) at the C-ABI's argument meaning ----
 * Strides are in elements. Weights (gamma, beta, w, wqk) are f32 arrays, as the reference stores them. */
void oracle_layernorm_f16(const uint16_t* x, int64_t xs, uint16_t* y, int64_t ys, const float* g,
                          const float* b, int64_t rows, int C, float eps);
void oracle_rmsnorm_f16(const uint16_t* x, int64_t xs, uint16_t* y, int64_t ys, const float* w,
                        int64_t rows, int C, float eps);
/* In place on the q and k heads of each qkv row (row = [q n_q*hd | k n_kv*hd | v ...], stride
 * row_stride). Position of row t is positions[t] if positions != NULL, else pos0 + t; rows whose
 * position is outside [0, n_pos) are left untouched. wqk = q_norm[hd] then k_norm[hd], or NULL to
 * skip the norm (rope.comp flags & 1). Follows qwen3_model.cpp:249-253 / rope.comp:25-51. */
void oracle_qk_norm_rope_f16(uint16_t* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                             int64_t pos0, const int32_t* positions, const float* wqk, const float* cs,
                             int64_t n_pos, float eps);
void oracle_qk_norm_rope_f32(float* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                             int64_t pos0, const int32_t* positions, const float* wqk, const float* cs,
                             int64_t n_pos, float eps);
/* KV store at the C ABI's argument meaning: k = qkv row + k_off, v = qkv row + v_off (width values
 * each), cache row = positions[t] or pos0 + t, rows outside [0, cache_rows) skipped; f16 activations
 * are copied bit for bit, f32 activations rounded to f16 (oracle_store_kv). */
void oracle_store_kv_rows(const void* qkv, int is_f16, int64_t row_stride, int64_t k_off, int64_t v_off, int width,
                          int64_t rows, int64_t pos0, const int32_t* positions, int64_t cache_rows, uint16_t* kc,
                          uint16_t* vc);
/* q/k norm + RoPE, then the KV store of the rotated keys and the values into cache row = the row's
 * position (qwen3_model.cpp:249-256); kc / vc rows are n_kv*hd halves; rows outside [0, n_pos) are
 * untouched and store nothing. */
void oracle_qk_norm_rope_kv_f16(uint16_t* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                                int64_t pos0, const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos,
                                float eps, uint16_t* kc, uint16_t* vc);
void oracle_qk_norm_rope_kv_f32(float* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd, int64_t pos0,
                                const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos, float eps,
                                uint16_t* kc, uint16_t* vc);
/* fp16 residual add + RMSNorm: x = f16(f32(x) + f32(d)) in place, then xn = rmsnorm_f16(x). */
void oracle_add_rmsnorm_f16(uint16_t* x, int64_t xs, const uint16_t* d, int64_t ds, uint16_t* xn, int64_t xns,
                            const float* w, int64_t rows, int C, float eps);
void oracle_swiglu_f16(const uint16_t* h, int64_t hs, uint16_t* out, int64_t os, int64_t rows, int I);
void oracle_gelu_f16(const uint16_t* x, uint16_t* y, int64_t n);
void oracle_gated_rmsnorm_f16(const uint16_t* y, int64_t ys, const uint16_t* z, int64_t zs, uint16_t* out,
                              int64_t os, const float* w, int64_t rows, int D, int groups, float eps);
/* Embedding gather (quant.cpp:230-253 + gpt2_model.cpp:182-187 / embed.comp): for each token t with
 * row = tokens[t] - row_base in [0, rows): out[t] = dequant(table row) (+ f32(wpe[pos0 + t]) when wpe
 * != NULL, added in f32). out_f16 != 0 rounds each f32 result once to f16; otherwise f32 is written.
 * Tokens outside the range leave their output row untouched. out rows have stride out_stride. */
void oracle_embed(const int32_t* tokens, int64_t T, const uint8_t* table, int64_t row_bytes, int fmt, int C,
                  int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t pos0, void* out,
                  int64_t out_stride, int out_f16);

/* Weight matmul, cpu::matmul on the portable path (cpu_ops.cpp:108-127 for F16 rows, :455-472 for FP8 /
 * FP4 rows): y[t][n] (+)= gelu?(x[t] . dequant(W[n]) + bias[n]) in float, k ascending; x is [T][K] f32,
 * W is N rows of row_bytes in `fmt`, y is [T][N]; flags 1 = gelu, 2 = accumulate into y. bias may be NULL. */
void oracle_matmul(int fmt, const float* x, int64_t T, int K, const uint8_t* w, int64_t row_bytes, int64_t N,
                   const float* bias, float* y, int flags);

#ifdef __cplusplus
}
#endif

#endif
