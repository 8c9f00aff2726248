// C entry points over the reference's own CPU ops, compiled from the reference sources where they lie
// (oracle/Makefile, target `ref`; output oracle/_ref/libneko_ref.so). TEST INFRASTRUCTURE ONLY: it
// pins the plain-C oracle and generates the golden fixtures; nothing in the product uses it.
//
// Everything arithmetic here is the reference's compiled code (neko::cpu::*, neko::quantizeMatrix,
// QMatrix::dequantizeRow, neko::f16_to_f32 / f32_to_f16). The only restated lines are the glue the
// reference has in files that do not build on x86 or need the whole model: the Granite gate
// (granite_model.cpp:21,282; that file includes <arm_neon.h> unconditionally), the Qwen3 per-token
// q/k loop (qwen3_model.cpp:249-253) and the GPT-2 wte+wpe add (gpt2_model.cpp:182-187).
#include <cmath>
#include <cstring>
#include <vector>

#include "common.h"
#include "cpu_ops.h"
#include "quant.h"

using namespace neko;

extern "C" {

float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t ref_f32_to_f16(float f) { return f32_to_f16(f); }

// Array forms: a scalar float return through a foreign-function layer quiets signalling NaNs.
void ref_f16_to_f32_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = f16_to_f32(h[i]);
}
void ref_f32_to_f16_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = f32_to_f16(f[i]);
}

float ref_gelu(float x) { return cpu::gelu(x); }

void ref_layernorm(const float* x, float* y, const float* g, const float* b, int T, int C, float eps) {
    cpu::layerNorm(x, y, g, b, T, C, eps);
}

void ref_rmsnorm(const float* x, float* y, const float* w, int rows, int C, float eps) {
    cpu::rmsNorm(x, y, w, rows, C, eps);
}

void ref_rope(float* x, int nHeads, int hd, const float* cs) { cpu::rope(x, nHeads, hd, cs); }

void ref_silu_mul(const float* h, float* out, int T, int I) { cpu::siluMul(h, out, T, I); }

size_t ref_quant_row_bytes(int fmt, int cols) { return quantRowBytes(WeightFormat(fmt), cols); }

// quantizeMatrix without a thread pool; returns the format actually used (F16 when cols % 32 != 0).
int ref_quantize_rows(int fmt, int rows, int cols, const float* src, uint8_t* dst) {
    QMatrix m = quantizeMatrix(
        WeightFormat(fmt), rows, cols,
        [&](int r, float* out) { std::memcpy(out, src + size_t(r) * size_t(cols), size_t(cols) * sizeof(float)); },
        nullptr);
    std::memcpy(dst, m.data.data(), m.data.size());
    return int(m.format);
}

void ref_dequantize_row(int fmt, int cols, const uint8_t* row, float* out) {
    QMatrix m;
    m.format = WeightFormat(fmt);
    m.rows = 1;
    m.cols = cols;
    m.rowBytes = quantRowBytes(m.format, cols);
    m.data.assign(row, row + m.rowBytes);
    m.dequantizeRow(0, out);
}

// ---- fp16 I/O compositions: reference widen -> reference op -> reference narrow.

static void widen(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; i++) f[i] = f16_to_f32(h[i]);
}
static void narrow(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = f32_to_f16(f[i]);
}

void ref_layernorm_f16(const uint16_t* x, uint16_t* y, const float* g, const float* b, int rows, int C, float eps) {
    std::vector<float> t(size_t(rows) * size_t(C)), o(t.size());
    widen(x, t.data(), t.size());
    cpu::layerNorm(t.data(), o.data(), g, b, rows, C, eps);
    narrow(o.data(), y, o.size());
}

void ref_rmsnorm_f16(const uint16_t* x, uint16_t* y, const float* w, int rows, int C, float eps) {
    std::vector<float> t(size_t(rows) * size_t(C)), o(t.size());
    widen(x, t.data(), t.size());
    cpu::rmsNorm(t.data(), o.data(), w, rows, C, eps);
    narrow(o.data(), y, o.size());
}

// Qwen3 attention prologue on rows of `stride` halves, positions[t] per row (qwen3_model.cpp:249-253).
void ref_qk_norm_rope_f16(uint16_t* qkv, int stride, int rows, int H, int KV, int hd, const int32_t* positions,
                          const float* qNorm, const float* kNorm, const float* cs, float eps) {
    const int width = (H + KV) * hd;
    std::vector<float> r(static_cast<size_t>(width));
    for (int t = 0; t < rows; t++) {
        uint16_t* row = qkv + size_t(t) * size_t(stride);
        widen(row, r.data(), r.size());
        if (qNorm) {
            cpu::rmsNorm(r.data(), r.data(), qNorm, H, hd, eps);
            cpu::rmsNorm(r.data() + H * hd, r.data() + H * hd, kNorm, KV, hd, eps);
        }
        cpu::rope(r.data(), H + KV, hd, cs + size_t(positions[t]) * size_t(hd));
        narrow(r.data(), row, r.size());
    }
}

void ref_silu_mul_f16(const uint16_t* h, uint16_t* out, int T, int I) {
    std::vector<float> t(size_t(T) * 2 * size_t(I)), o(size_t(T) * size_t(I));
    widen(h, t.data(), t.size());
    cpu::siluMul(t.data(), o.data(), T, I);
    narrow(o.data(), out, o.size());
}

void ref_gelu_f16(const uint16_t* x, uint16_t* y, int n) {
    for (int i = 0; i < n; i++) y[i] = f32_to_f16(cpu::gelu(f16_to_f32(x[i])));
}

// Granite gate + group norm: the gate is restated (granite_model.cpp:21,282), the norm is the compiled
// cpu::rmsNorm applied per group exactly as granite_model.cpp:283-285 does.
void ref_gated_rmsnorm_f16(const uint16_t* y, const uint16_t* z, uint16_t* out, const float* w, int rows, int D,
                           int groups, float eps) {
    const int GS = D / groups;
    std::vector<float> yr(static_cast<size_t>(D)), zr(static_cast<size_t>(D));
    for (int t = 0; t < rows; t++) {
        widen(y + size_t(t) * size_t(D), yr.data(), yr.size());
        widen(z + size_t(t) * size_t(D), zr.data(), zr.size());
        for (int i = 0; i < D; i++) yr[size_t(i)] *= zr[size_t(i)] / (1.0f + std::exp(-zr[size_t(i)]));
        for (int g = 0; g < groups; g++)
            cpu::rmsNorm(yr.data() + size_t(g) * size_t(GS), yr.data() + size_t(g) * size_t(GS), w + size_t(g) * size_t(GS),
                         1, GS, eps);
        narrow(yr.data(), out + size_t(t) * size_t(D), yr.size());
    }
}

// KV-cache store: the compiled cpu::storeKv.
void ref_store_kv(const float* k, const float* v, int src_stride, uint16_t* kc, uint16_t* vc, int width, int T, int pos0) {
    cpu::storeKv(k, v, src_stride, kc, vc, width, T, pos0);
}

// Causal grouped-query attention: the compiled cpu::attention on a one-thread pool.
void ref_attention(const float* q, int q_stride, const uint16_t* kc, const uint16_t* vc, float* out, int T, int n_head,
                   int n_kv, int hd, int pos0) {
    static ThreadPool pool(1);
    cpu::attention(pool, q, q_stride, kc, vc, out, T, n_head, n_kv, hd, pos0);
}

// Residual add + RMSNorm with f16 I/O, entirely through compiled reference code: the add is the
// matmulF16 kAccumulate epilogue (cpu_ops.cpp:123) with an identity weight matrix, so each output
// row is y = y + (sum of 1 * d[n] and exact zeros) = y + d (finite d); then cpu::rmsNorm of the
// f16-rounded sum. x_out receives the rounded sum.
void ref_add_rmsnorm_f16(const uint16_t* x, const uint16_t* d, uint16_t* x_out, uint16_t* xn, const float* w, int rows,
                         int C, float eps) {
    std::vector<float> xs(size_t(rows) * size_t(C)), ds(xs.size()), y(xs.size());
    widen(x, xs.data(), xs.size());
    widen(d, ds.data(), ds.size());
    std::vector<uint16_t> eye(size_t(C) * size_t(C), 0);
    for (int n = 0; n < C; n++) eye[size_t(n) * size_t(C) + size_t(n)] = 0x3C00;  // 1.0
    ThreadPool pool(1);
    cpu::matmulF16(pool, ds.data(), rows, C, eye.data(), nullptr, xs.data(), C, cpu::kAccumulate);
    narrow(xs.data(), x_out, xs.size());
    widen(x_out, xs.data(), xs.size());
    cpu::rmsNorm(xs.data(), y.data(), w, rows, C, eps);
    narrow(y.data(), xn, y.size());
}

// Weight matmul: the compiled cpu::matmul on a one-thread pool (x86: matmulF16 for F16 rows,
// matmulGeneric for FP8 / FP4).
void ref_matmul(int fmt, const float* x, int T, int K, const uint8_t* table, int N, const float* bias, float* y,
                int flags) {
    QMatrix m;
    m.format = WeightFormat(fmt);
    m.rows = N;
    m.cols = K;
    m.rowBytes = quantRowBytes(m.format, K);
    m.data.assign(table, table + m.rowBytes * size_t(N));
    static ThreadPool pool(1);
    cpu::matmul(pool, x, T, K, m, bias, y, N, flags);
}

// ---- f32 activations, as the reference's CPU forward passes hold them (its CPU path, timed beside
// the device kernels; same compiled ops, no f16 widening or narrowing).

// GELU over n values: what the matmul epilogue applies per output under kGelu (cpu_ops.cpp:121,143).
void ref_gelu_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = cpu::gelu(x[i]);
}

// The Qwen3 per-token q/k norm + RoPE loop on f32 rows of `stride` floats (qwen3_model.cpp:249-253).
void ref_qk_norm_rope(float* qkv, int stride, int rows, int H, int KV, int hd, const int32_t* positions,
                      const float* qNorm, const float* kNorm, const float* cs, float eps) {
    const int kOff = H * hd;
    for (int t = 0; t < rows; t++) {
        float* r = qkv + size_t(t) * size_t(stride);
        cpu::rmsNorm(r, r, qNorm, H, hd, eps);
        cpu::rmsNorm(r + kOff, r + kOff, kNorm, KV, hd, eps);
        cpu::rope(r, H + KV, hd, cs + size_t(positions[t]) * size_t(hd));
    }
}

// The Granite gate + group norm in place on f32 rows (granite_model.cpp:21,278-285).
void ref_gated_rmsnorm(float* y, const float* z, const float* w, int rows, int D, int groups, float eps) {
    const int GS = D / groups;
    for (int t = 0; t < rows; t++) {
        float* yr = y + size_t(t) * size_t(D);
        const float* zr = z + size_t(t) * size_t(D);
        for (int i = 0; i < D; i++) yr[i] *= zr[i] / (1.0f + std::exp(-zr[i]));
        for (int g = 0; g < groups; g++)
            cpu::rmsNorm(yr + size_t(g) * size_t(GS), yr + size_t(g) * size_t(GS), w + size_t(g) * size_t(GS), 1, GS, eps);
    }
}

// A weight table held as the reference's QMatrix, so a gather can be timed without copying the table
// per call: the embedding loop dequantizeRow(tokens[t]) into f32 rows (qwen3_model.cpp:236), plus,
// when wpe (T f32 position rows) is given, GPT-2's position add (gpt2_model.cpp:182-187).
void* ref_qmatrix_new(int fmt, int rows, int C, const uint8_t* table) {
    QMatrix* m = new QMatrix();
    m->format = WeightFormat(fmt);
    m->rows = rows;
    m->cols = C;
    m->rowBytes = quantRowBytes(m->format, C);
    m->data.assign(table, table + m->rowBytes * size_t(rows));
    return m;
}
void ref_qmatrix_gather(const void* h, const int32_t* tokens, int T, const float* wpe, float* out) {
    const QMatrix* m = static_cast<const QMatrix*>(h);
    const int C = m->cols;
    for (int t = 0; t < T; t++) {
        float* xr = out + size_t(t) * size_t(C);
        m->dequantizeRow(tokens[t], xr);
        if (wpe) {
            const float* pe = wpe + size_t(t) * size_t(C);
            for (int c = 0; c < C; c++) xr[c] += pe[c];
        }
    }
}
void ref_qmatrix_free(void* h) { delete static_cast<QMatrix*>(h); }
// cpu::matmul over a held QMatrix (no per-call copy of the table), one-thread pool.
void ref_qmatrix_matmul(const void* h, const float* x, int T, const float* bias, float* y, int flags) {
    const QMatrix* m = static_cast<const QMatrix*>(h);
    static ThreadPool pool(1);
    cpu::matmul(pool, x, T, m->cols, *m, bias, y, m->rows, flags);
}

// Embedding gather: dequantizeRow of each token's row, + the f32 position row (gpt2_model.cpp:182-187),
// rounded to f16 when out_f16.
void ref_embed(const int32_t* tokens, int T, const uint8_t* table, int fmt, int rows, int C, const uint16_t* wpe,
               int pos0, void* out, int out_f16) {
    QMatrix m;
    m.format = WeightFormat(fmt);
    m.rows = rows;
    m.cols = C;
    m.rowBytes = quantRowBytes(m.format, C);
    m.data.assign(table, table + m.rowBytes * size_t(rows));
    std::vector<float> x(static_cast<size_t>(C));
    for (int t = 0; t < T; t++) {
        m.dequantizeRow(tokens[t], x.data());
        if (wpe)
            for (int c = 0; c < C; c++) x[size_t(c)] += f16_to_f32(wpe[size_t(pos0 + t) * size_t(C) + size_t(c)]);
        if (out_f16) narrow(x.data(), static_cast<uint16_t*>(out) + size_t(t) * size_t(C), x.size());
        else std::memcpy(static_cast<float*>(out) + size_t(t) * size_t(C), x.data(), x.size() * sizeof(float));
    }
}

}  // extern "C"
