/*
 * CPU oracle: plain-C restatement of the reference's fused-layer-op arithmetic.
 * TEST INFRASTRUCTURE ONLY -- see neko_oracle.h for scope, citations and how each part is pinned.
 *
 * Build: no -march (x86-64 baseline, SSE2 float arithmetic, no FMA instructions) and
 * -ffp-contract=off, so every float expression rounds exactly where the reference's portable path
 * (compiled with g++ -O3, CMakeLists.txt:99) rounds.
 */
#include "neko_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 helpers */

/* Exact widening, subnormals included (common.h:33-55). */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        /* value m * 2^-24: move the leading one up to bit 10, lowering the exponent per step */
        uint32_t exp32 = 113u;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            exp32--;
        }
        bits = sign | (exp32 << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even narrowing; overflow -> inf, NaN -> sign | 0x7E00, underflow -> signed zero
 * (common.h:57-80). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e32 = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e32 == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
    int e = (int)e32 - 112; /* biased f16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = m | 0x800000u;
        uint32_t sh = (uint32_t)(14 - e);
        uint32_t q = full >> sh;
        uint32_t rem = full & ((1u << sh) - 1u);
        uint32_t tie = 1u << (sh - 1u);
        if (rem > tie || (rem == tie && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = sign | ((uint32_t)e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)q;
}

float oracle_bf16_to_f32(uint16_t b) { /* common.h:82-87 */
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void oracle_f16_to_f32_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = oracle_f16_to_f32(h[i]);
}

void oracle_f32_to_f16_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = oracle_f32_to_f16(f[i]);
}

/* ------------------------------------------------------------------ f32 ops */

/* GPT-2 "gelu_new", tanh form, evaluated left to right in float (cpu_ops.cpp:20-23). */
float oracle_gelu(float x) {
    const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* Two-pass LayerNorm with double accumulators; output in float, left to right
 * (cpu_ops.cpp:483-500). */
void oracle_layernorm(const float* x, float* y, const float* g, const float* b, int rows, int C, float eps) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * (size_t)C;
        float* yr = y + (size_t)r * (size_t)C;
        double mean = 0.0;
        for (int c = 0; c < C; c++) mean += xr[c];
        mean /= C;
        double var = 0.0;
        for (int c = 0; c < C; c++) {
            double d = xr[c] - mean;
            var += d * d;
        }
        var /= C;
        const float rs = (float)(1.0 / sqrt(var + eps));
        const float m = (float)mean;
        for (int c = 0; c < C; c++) yr[c] = (xr[c] - m) * rs * g[c] + b[c];
    }
}

/* RMSNorm: double sum of squares, float scale, y = x * s * w; y may alias x (cpu_ops.cpp:502-511). */
void oracle_rmsnorm(const float* x, float* y, const float* w, int rows, int C, float eps) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * (size_t)C;
        float* yr = y + (size_t)r * (size_t)C;
        double ss = 0.0;
        for (int c = 0; c < C; c++) ss += (double)xr[c] * xr[c];
        const float s = (float)(1.0 / sqrt(ss / C + eps));
        for (int c = 0; c < C; c++) yr[c] = xr[c] * s * w[c];
    }
}

/* NeoX half-split rotation of n_heads consecutive heads; cs = hd/2 (cos, sin) pairs
 * (cpu_ops.cpp:513-524). */
void oracle_rope(float* x, int n_heads, int hd, const float* cs) {
    const int half = hd / 2;
    for (int h = 0; h < n_heads; h++) {
        float* v = x + (size_t)h * (size_t)hd;
        for (int i = 0; i < half; i++) {
            const float c = cs[2 * i], s = cs[2 * i + 1];
            const float a = v[i], bb = v[i + half];
            v[i] = a * c - bb * s;
            v[i + half] = a * s + bb * c;
        }
    }
}

/* SwiGLU over rows holding [gate I | up I] (cpu_ops.cpp:526-533). */
void oracle_silu_mul(const float* h, float* out, int rows, int I) {
    for (int t = 0; t < rows; t++) {
        const float* gate = h + (size_t)t * 2u * (size_t)I;
        const float* up = gate + I;
        float* o = out + (size_t)t * (size_t)I;
        for (int i = 0; i < I; i++) o[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
    }
}

float oracle_silu(float v) { return v / (1.0f + expf(-v)); } /* granite_model.cpp:21 */

/* Granite-4.0-H Mamba2 output gate + group RMSNorm, in place on y (granite_model.cpp:278-287). */
void oracle_gated_rmsnorm(float* y, const float* z, int64_t z_stride, const float* w, int rows, int D, int groups,
                          float eps) {
    const int GS = D / groups;
    for (int t = 0; t < rows; t++) {
        float* yr = y + (size_t)t * (size_t)D;
        const float* zr = z + (size_t)t * (size_t)z_stride;
        for (int i = 0; i < D; i++) yr[i] *= oracle_silu(zr[i]);
        for (int g = 0; g < groups; g++)
            oracle_rmsnorm(yr + (size_t)g * (size_t)GS, yr + (size_t)g * (size_t)GS, w + (size_t)g * (size_t)GS, 1, GS,
                           eps);
    }
}

/* KV-cache store (cpu_ops.cpp:535-542): row t's k and v, width floats each, rounded to f16 into cache
 * row pos0 + t (toHalf, cpu_ops.cpp:98-104). */
void oracle_store_kv(const float* k, const float* v, int64_t src_stride, uint16_t* kc, uint16_t* vc, int width,
                     int64_t T, int64_t pos0) {
    for (int64_t t = 0; t < T; t++) {
        const int64_t dst = (pos0 + t) * (int64_t)width;
        oracle_f32_to_f16_n(k + t * src_stride, kc + dst, width);
        oracle_f32_to_f16_n(v + t * src_stride, vc + dst, width);
    }
}

/* Causal grouped-query attention (cpu_ops.cpp:544-575): for token t (position pos0 + t) and head h,
 * over cache rows j = 0 .. pos0 + t: s_j = (sum over d, in d order, of q[d] * k_j[d]) * scale, scale =
 * 1 / sqrtf(hd); mx = the largest s_j; e_j = expf(s_j - mx), summed in j order; acc[d] = sum over j, in j
 * order, of e_j * v_j[d]; out[d] = acc[d] * (1 / sum). k_j / v_j: kv head h / (n_head / n_kv) of cache
 * row j (rows of n_kv * hd halves); out rows are n_head * hd floats. */
void oracle_attention(const float* q, int64_t q_stride, const uint16_t* kc, const uint16_t* vc, float* out, int64_t T,
                      int n_head, int n_kv, int hd, int64_t pos0) {
    const int64_t kvw = (int64_t)n_kv * hd;
    const int group = n_head / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    float* scores = malloc(sizeof(float) * (size_t)(pos0 + T));
    float* acc = malloc(sizeof(float) * (size_t)hd);
    if (!scores || !acc) abort();
    for (int64_t t = 0; t < T; t++) {
        for (int h = 0; h < n_head; h++) {
            const int64_t L = pos0 + t + 1;
            const float* qh = q + t * q_stride + (int64_t)h * hd;
            const int64_t off = (int64_t)(h / group) * hd;
            float mx = -INFINITY;
            for (int64_t j = 0; j < L; j++) {
                const uint16_t* kr = kc + j * kvw + off;
                float s = 0.0f;
                for (int d = 0; d < hd; d++) s += qh[d] * oracle_f16_to_f32(kr[d]);
                s = s * scale;
                scores[j] = s;
                mx = mx < s ? s : mx; /* std::max(mx, s) */
            }
            float sum = 0.0f;
            for (int64_t j = 0; j < L; j++) {
                const float e = expf(scores[j] - mx);
                scores[j] = e;
                sum += e;
            }
            for (int d = 0; d < hd; d++) acc[d] = 0.0f;
            for (int64_t j = 0; j < L; j++) {
                const uint16_t* vr = vc + j * kvw + off;
                for (int d = 0; d < hd; d++) acc[d] += scores[j] * oracle_f16_to_f32(vr[d]);
            }
            const float inv = 1.0f / sum;
            float* o = out + t * (int64_t)n_head * hd + (int64_t)h * hd;
            for (int d = 0; d < hd; d++) o[d] = acc[d] * inv;
        }
    }
    free(scores);
    free(acc);
}

/* Residual add then RMSNorm: the matmul epilogue with kAccumulate adds the product into the residual
 * row, dst = dst + v in float (cpu_ops.cpp:123), and the next op norms that row (qwen3_model.cpp:264,
 * cpu_ops.cpp:502-511). Here v is the delta row d. */
void oracle_add_rmsnorm(float* x, const float* d, float* xn, const float* w, int rows, int C, float eps) {
    for (int t = 0; t < rows; t++) {
        float* xr = x + (size_t)t * (size_t)C;
        const float* dr = d + (size_t)t * (size_t)C;
        for (int i = 0; i < C; i++) xr[i] = xr[i] + dr[i];
        oracle_rmsnorm(xr, xn + (size_t)t * (size_t)C, w, 1, C, eps);
    }
}

/* RoPE table in double, stored as float pairs (qwen3_model.cpp:102-114). */
void oracle_rope_table(double theta, int hd, int n_pos, float* cs) {
    for (int i = 0; i < hd / 2; i++) {
        const double inv = pow(theta, -2.0 * i / hd);
        for (int p = 0; p < n_pos; p++) {
            const double a = p * inv;
            cs[(size_t)p * (size_t)hd + (size_t)(2 * i)] = (float)cos(a);
            cs[(size_t)p * (size_t)hd + (size_t)(2 * i + 1)] = (float)sin(a);
        }
    }
}

/* ------------------------------------------------------------------ weight formats */

enum { kBlock = 32 };

size_t oracle_quant_row_bytes(int fmt, int cols) { /* quant.cpp:199-208 */
    const size_t c = (size_t)cols;
    const size_t scale_bytes = ((c / kBlock) * 2u + 15u) / 16u * 16u;
    switch (fmt) {
        case ORACLE_FMT_F16: return c * 2u;
        case ORACLE_FMT_FP8: return c + scale_bytes;
        case ORACLE_FMT_FP4: return c / 2u + scale_bytes;
    }
    return 0;
}

/* E4M3 code -> f16 bit pattern (value / 256), times 256 (quant.cpp:51-53). */
float oracle_decode_fp8(uint8_t c) {
    const uint16_t bits = (uint16_t)(((c & 0x80u) << 8) | ((c & 0x7fu) << 7));
    return oracle_f16_to_f32(bits) * 256.0f;
}

/* E2M1 code -> f16 bit pattern (value / 16384), times 16384 (quant.cpp:63-65). */
float oracle_decode_fp4(uint8_t c) {
    const uint16_t bits = (uint16_t)(((c & 8u) << 12) | ((c & 7u) << 9));
    return oracle_f16_to_f32(bits) * 16384.0f;
}

/* quant.cpp:43-49: RNE of the f16 pattern of y/256 over its 7 low bits, clamped to 0x7E (448). */
uint8_t oracle_encode_fp8(float y) {
    const uint16_t h = oracle_f32_to_f16(y * (1.0f / 256.0f));
    const uint32_t mag = h & 0x7fffu;
    uint32_t code = (mag + 0x3fu + ((mag >> 7) & 1u)) >> 7;
    if (code > 0x7eu) code = 0x7eu;
    return (uint8_t)(code | ((h >> 8) & 0x80u));
}

/* quant.cpp:57-61: threshold ladder over |y|; zero magnitude never carries a sign. */
uint8_t oracle_encode_fp4(float y) {
    const float a = fabsf(y);
    const int c = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.0f);
    return (uint8_t)(c == 0 ? 0 : (c | (y < 0 ? 8 : 0)));
}

/* max over |x| with std::max semantics (a NaN never replaces the running maximum). */
static float block_amax(const float* x) {
    float amax = 0.0f;
    for (int i = 0; i < kBlock; i++) {
        const float a = fabsf(x[i]);
        if (amax < a) amax = a;
    }
    return amax;
}

/* quant.cpp:72-79 */
static uint16_t block_scale(const float* x, float max_code, float* inv) {
    const uint16_t s = oracle_f32_to_f16(block_amax(x) / max_code);
    const float sv = oracle_f16_to_f32(s);
    *inv = sv > 0 ? 1.0f / sv : 0.0f;
    return sv > 0 ? s : 0;
}

/* quant.cpp:93-97 */
static float fp4_round(float a) {
    if (a < 1.75f) return nearbyintf(a * 2.0f) * 0.5f;
    if (a < 3.5f) return nearbyintf(a);
    return a < 5.0f ? 4.0f : 6.0f;
}

typedef struct {
    float err, xr, rr;
} fp4_fit;

/* Portable (non-NEON) branch, sequential float sums (quant.cpp:126-137). */
static fp4_fit fit_fp4(const float* ax, float s) {
    fp4_fit f = {0.0f, 0.0f, 0.0f};
    const float inv = 1.0f / s;
    for (int i = 0; i < kBlock; i++) {
        const float r = fp4_round(ax[i] * inv);
        const float d = ax[i] - r * s;
        f.err += d * d;
        f.xr += ax[i] * r;
        f.rr += r * r;
    }
    return f;
}

/* Start at amax/6, then up to two least-squares refits kept only while the error drops
 * (quant.cpp:142-165). */
uint16_t oracle_fp4_block_scale(const float* xb) {
    uint16_t best = oracle_f32_to_f16(block_amax(xb) / 6.0f);
    if (oracle_f16_to_f32(best) <= 0) return 0;
    float ax[kBlock];
    for (int i = 0; i < kBlock; i++) ax[i] = fabsf(xb[i]);
    fp4_fit fit = fit_fp4(ax, oracle_f16_to_f32(best));
    float best_err = fit.err;
    for (int iter = 0; iter < 2 && fit.rr > 0; iter++) {
        const uint16_t s = oracle_f32_to_f16(fit.xr / fit.rr);
        if (oracle_f16_to_f32(s) <= 0 || s == best) break;
        fit = fit_fp4(ax, oracle_f16_to_f32(s));
        if (fit.err >= best_err) break;
        best_err = fit.err;
        best = s;
    }
    return best;
}

static void put_u16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xffu);
    p[1] = (uint8_t)(v >> 8);
}

static uint16_t get_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static void quantize_row_fp8(const float* x, int cols, uint8_t* out) { /* quant.cpp:81-90 */
    for (int b = 0; b < cols / kBlock; b++) {
        const float* xb = x + b * kBlock;
        float inv;
        put_u16(out + cols + 2 * b, block_scale(xb, 448.0f, &inv));
        for (int i = 0; i < kBlock; i++) out[b * kBlock + i] = oracle_encode_fp8(xb[i] * inv);
    }
}

static void quantize_row_fp4(const float* x, int cols, uint8_t* out) { /* quant.cpp:167-178 */
    for (int b = 0; b < cols / kBlock; b++) {
        const float* xb = x + b * kBlock;
        const uint16_t s = oracle_fp4_block_scale(xb);
        put_u16(out + cols / 2 + 2 * b, s);
        const float inv = s ? 1.0f / oracle_f16_to_f32(s) : 0.0f;
        uint8_t* o = out + b * (kBlock / 2);
        for (int j = 0; j < 16; j++)
            o[j] = (uint8_t)(oracle_encode_fp4(xb[j] * inv) | (oracle_encode_fp4(xb[16 + j] * inv) << 4));
    }
}

int oracle_quantize_rows(int fmt, int64_t rows, int cols, const float* src, uint8_t* dst) {
    if (cols % kBlock != 0) fmt = ORACLE_FMT_F16; /* quant.cpp:257 */
    const size_t rb = oracle_quant_row_bytes(fmt, cols);
    memset(dst, 0, rb * (size_t)rows);
    for (int64_t r = 0; r < rows; r++) {
        const float* x = src + (size_t)r * (size_t)cols;
        uint8_t* out = dst + (size_t)r * rb;
        if (fmt == ORACLE_FMT_F16) {
            for (int c = 0; c < cols; c++) put_u16(out + 2 * c, oracle_f32_to_f16(x[c])); /* quant.cpp:180-186 */
        } else if (fmt == ORACLE_FMT_FP8) {
            quantize_row_fp8(x, cols, out);
        } else {
            quantize_row_fp4(x, cols, out);
        }
    }
    return fmt;
}

void oracle_dequantize_row(int fmt, int cols, const uint8_t* p, float* out) { /* quant.cpp:230-253 */
    if (fmt == ORACLE_FMT_F16) {
        for (int c = 0; c < cols; c++) out[c] = oracle_f16_to_f32(get_u16(p + 2 * c));
    } else if (fmt == ORACLE_FMT_FP8) {
        for (int c = 0; c < cols; c++)
            out[c] = oracle_decode_fp8(p[c]) * oracle_f16_to_f32(get_u16(p + cols + 2 * (c / kBlock)));
    } else {
        for (int c = 0; c < cols; c++) {
            const int b = c / kBlock, j = c % kBlock;
            const uint8_t byte = p[b * 16 + (j & 15)];
            const uint8_t code = (uint8_t)(j < 16 ? (byte & 0xfu) : (byte >> 4));
            out[c] = oracle_decode_fp4(code) * oracle_f16_to_f32(get_u16(p + cols / 2 + 2 * b));
        }
    }
}

/* ------------------------------------------------------------------ fp16 I/O compositions */

static float* scratch_f32(size_t n) {
    float* p = (float*)malloc((n ? n : 1) * sizeof(float));
    if (!p) abort();
    return p;
}

void oracle_layernorm_f16(const uint16_t* x, int64_t xs, uint16_t* y, int64_t ys, const float* g, const float* b,
                          int64_t rows, int C, float eps) {
    float* t = scratch_f32((size_t)C);
    for (int64_t r = 0; r < rows; r++) {
        oracle_f16_to_f32_n(x + r * xs, t, C);
        oracle_layernorm(t, t, g, b, 1, C, eps);
        oracle_f32_to_f16_n(t, y + r * ys, C);
    }
    free(t);
}

void oracle_rmsnorm_f16(const uint16_t* x, int64_t xs, uint16_t* y, int64_t ys, const float* w, int64_t rows, int C,
                        float eps) {
    float* t = scratch_f32((size_t)C);
    for (int64_t r = 0; r < rows; r++) {
        oracle_f16_to_f32_n(x + r * xs, t, C);
        oracle_rmsnorm(t, t, w, 1, C, eps);
        oracle_f32_to_f16_n(t, y + r * ys, C);
    }
    free(t);
}

/* One qkv row in f32: q heads then k heads normed with their own weights, then all rotated
 * (qwen3_model.cpp:249-253; the no-norm form is rope.comp with flags = 0). */
static void qk_row_f32(float* t, int n_q, int n_kv, int hd, const float* wqk, const float* cs_row, float eps) {
    if (wqk) {
        oracle_rmsnorm(t, t, wqk, n_q, hd, eps);
        oracle_rmsnorm(t + (size_t)n_q * (size_t)hd, t + (size_t)n_q * (size_t)hd, wqk + hd, n_kv, hd, eps);
    }
    oracle_rope(t, n_q + n_kv, hd, cs_row);
}

static int row_position(int64_t t, int64_t pos0, const int32_t* positions, int64_t n_pos, int64_t* pos) {
    const int64_t p = positions ? (int64_t)positions[t] : pos0 + t;
    *pos = p;
    return p >= 0 && p < n_pos;
}

void oracle_qk_norm_rope_f16(uint16_t* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd, int64_t pos0,
                             const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos, float eps) {
    const int64_t width = (int64_t)(n_q + n_kv) * hd;
    float* t = scratch_f32((size_t)width);
    for (int64_t r = 0; r < rows; r++) {
        int64_t pos;
        if (!row_position(r, pos0, positions, n_pos, &pos)) continue;
        uint16_t* row = qkv + r * row_stride;
        oracle_f16_to_f32_n(row, t, width);
        qk_row_f32(t, n_q, n_kv, hd, wqk, cs + pos * hd, eps);
        oracle_f32_to_f16_n(t, row, width);
    }
    free(t);
}

void oracle_qk_norm_rope_f32(float* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd, int64_t pos0,
                             const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        int64_t pos;
        if (!row_position(r, pos0, positions, n_pos, &pos)) continue;
        qk_row_f32(qkv + r * row_stride, n_q, n_kv, hd, wqk, cs + pos * hd, eps);
    }
}

/* The KV store at the C ABI's argument meaning: cache row = positions[t] (or pos0 + t); rows whose
 * cache row is outside [0, cache_rows) are skipped. f16 activations are copied bit for bit (a
 * half widened to f32 and rounded back is itself); f32 activations are rounded by
 * oracle_store_kv. */
void oracle_store_kv_rows(const void* qkv, int is_f16, int64_t row_stride, int64_t k_off, int64_t v_off, int width,
                          int64_t rows, int64_t pos0, const int32_t* positions, int64_t cache_rows, uint16_t* kc,
                          uint16_t* vc) {
    for (int64_t t = 0; t < rows; t++) {
        int64_t p;
        if (!row_position(t, pos0, positions, cache_rows, &p)) continue;
        if (is_f16) {
            const uint16_t* r = (const uint16_t*)qkv + t * row_stride;
            memcpy(kc + p * width, r + k_off, (size_t)width * 2u);
            memcpy(vc + p * width, r + v_off, (size_t)width * 2u);
        } else {
            const float* r = (const float*)qkv + t * row_stride;
            oracle_store_kv(r + k_off, r + v_off, 0, kc, vc, width, 1, p);
        }
    }
}

/* q/k norm + RoPE then the KV store of the rotated keys and the values (qwen3_model.cpp:249-256),
 * cache row = the row's position; rows outside [0, n_pos) are left untouched and store nothing. */
void oracle_qk_norm_rope_kv_f16(uint16_t* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd,
                                int64_t pos0, const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos,
                                float eps, uint16_t* kc, uint16_t* vc) {
    oracle_qk_norm_rope_f16(qkv, row_stride, rows, n_q, n_kv, hd, pos0, positions, wqk, cs, n_pos, eps);
    const int64_t kw = (int64_t)n_kv * hd;
    oracle_store_kv_rows(qkv, 1, row_stride, (int64_t)n_q * hd, (int64_t)n_q * hd + kw, (int)kw, rows, pos0, positions,
                         n_pos, kc, vc);
}

void oracle_qk_norm_rope_kv_f32(float* qkv, int64_t row_stride, int64_t rows, int n_q, int n_kv, int hd, int64_t pos0,
                                const int32_t* positions, const float* wqk, const float* cs, int64_t n_pos, float eps,
                                uint16_t* kc, uint16_t* vc) {
    oracle_qk_norm_rope_f32(qkv, row_stride, rows, n_q, n_kv, hd, pos0, positions, wqk, cs, n_pos, eps);
    const int64_t kw = (int64_t)n_kv * hd;
    oracle_store_kv_rows(qkv, 0, row_stride, (int64_t)n_q * hd, (int64_t)n_q * hd + kw, (int)kw, rows, pos0, positions,
                         n_pos, kc, vc);
}

/* fp16 residual add + RMSNorm: x = f16(f32(x) + f32(d)) stored back, then xn = rmsnorm of the stored
 * halves (the unfused add-then-norm sequence with fp16 activations). */
void oracle_add_rmsnorm_f16(uint16_t* x, int64_t xs, const uint16_t* d, int64_t ds, uint16_t* xn, int64_t xns,
                            const float* w, int64_t rows, int C, float eps) {
    float* t = scratch_f32((size_t)2 * (size_t)C);
    for (int64_t r = 0; r < rows; r++) {
        oracle_f16_to_f32_n(x + r * xs, t, C);
        oracle_f16_to_f32_n(d + r * ds, t + C, C);
        for (int i = 0; i < C; i++) t[i] = t[i] + t[C + i];
        oracle_f32_to_f16_n(t, x + r * xs, C);
    }
    free(t);
    oracle_rmsnorm_f16(x, xs, xn, xns, w, rows, C, eps);
}

void oracle_swiglu_f16(const uint16_t* h, int64_t hs, uint16_t* out, int64_t os, int64_t rows, int I) {
    float* t = scratch_f32((size_t)3 * (size_t)I);
    for (int64_t r = 0; r < rows; r++) {
        oracle_f16_to_f32_n(h + r * hs, t, 2 * (int64_t)I);
        oracle_silu_mul(t, t + 2 * (size_t)I, 1, I);
        oracle_f32_to_f16_n(t + 2 * (size_t)I, out + r * os, I);
    }
    free(t);
}

void oracle_gelu_f16(const uint16_t* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = oracle_f32_to_f16(oracle_gelu(oracle_f16_to_f32(x[i])));
}

void oracle_gated_rmsnorm_f16(const uint16_t* y, int64_t ys, const uint16_t* z, int64_t zs, uint16_t* out, int64_t os,
                              const float* w, int64_t rows, int D, int groups, float eps) {
    float* t = scratch_f32((size_t)2 * (size_t)D);
    for (int64_t r = 0; r < rows; r++) {
        oracle_f16_to_f32_n(y + r * ys, t, D);
        oracle_f16_to_f32_n(z + r * zs, t + D, D);
        oracle_gated_rmsnorm(t, t + D, D, w, 1, D, groups, eps);
        oracle_f32_to_f16_n(t, out + r * os, D);
    }
    free(t);
}

void oracle_embed(const int32_t* tokens, int64_t T, const uint8_t* table, int64_t row_bytes, int fmt, int C,
                  int64_t row_base, int64_t rows, const uint16_t* wpe, int64_t pos0, void* out, int64_t out_stride,
                  int out_f16) {
    float* t = scratch_f32((size_t)C);
    for (int64_t i = 0; i < T; i++) {
        const int64_t row = (int64_t)tokens[i] - row_base;
        if (row < 0 || row >= rows) continue;
        oracle_dequantize_row(fmt, C, table + row * row_bytes, t);
        if (wpe) {
            const uint16_t* pe = wpe + (pos0 + i) * (int64_t)C;
            for (int c = 0; c < C; c++) t[c] += oracle_f16_to_f32(pe[c]);
        }
        if (out_f16)
            oracle_f32_to_f16_n(t, (uint16_t*)out + i * out_stride, C);
        else
            memcpy((float*)out + i * out_stride, t, (size_t)C * sizeof(float));
    }
    free(t);
}

/* ------------------------------------------------------------------ weight matmul */

/* cpu::matmul on the portable (non-aarch64) path, cpu_ops.cpp:474-490. F16 rows go through matmulF16
 * (:108-127): the dot starts at 0 and runs k = 0..K-1 in float (dotRow4's scalar loop, :60-63), then
 * v = dot + bias. FP8 / FP4 rows go through matmulGeneric (:455-472): dequantizeRow, then the sum starts
 * at the bias and adds x[k] * w[k] for k = 0..K-1. Both then apply gelu (flags & 1) and add into y
 * (flags & 2); y rows have stride N. */
void oracle_matmul(int fmt, const float* x, int64_t T, int K, const uint8_t* w, int64_t row_bytes, int64_t N,
                   const float* bias, float* y, int flags) {
    float* wr = scratch_f32((size_t)K);
    for (int64_t n = 0; n < N; n++) {
        oracle_dequantize_row(fmt, K, w + n * row_bytes, wr);
        for (int64_t t = 0; t < T; t++) {
            const float* xt = x + t * (int64_t)K;
            float v;
            if (fmt == ORACLE_FMT_F16) {
                float acc = 0.0f;
                for (int k = 0; k < K; k++) acc += wr[k] * xt[k];
                v = acc + (bias ? bias[n] : 0.0f);
            } else {
                v = bias ? bias[n] : 0.0f;
                for (int k = 0; k < K; k++) v += xt[k] * wr[k];
            }
            if (flags & 1) v = oracle_gelu(v);
            float* dst = y + t * N + n;
            *dst = (flags & 2) ? *dst + v : v;
        }
    }
    free(wr);
}
