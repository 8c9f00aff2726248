// Host-side weight codecs and RoPE table: the load-time half of the path, producing exactly the bytes
// and floats the reference's loader produces (quant.cpp:199-279 portable branch,
// qwen3_model.cpp:102-114), so tables encoded here gather bit-exactly with the reference's.
//
// Built without -march and with -ffp-contract=off: float arithmetic is plain SSE2 single precision
// with every product and sum rounded separately, as in the reference's x86 build.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/neko_hip.h"

namespace {

constexpr int kBlock = 32;

// IEEE binary16 from float, round-to-nearest-even; NaN -> sign | 0x7E00 (common.h:57-80 semantics).
uint16_t to_half_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t biased = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (biased == 0xffu) return static_cast<uint16_t>(sign | 0x7c00u | (mant ? 0x200u : 0u));
    const int e = static_cast<int>(biased) - 127 + 15;
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        mant |= 0x800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - e);
        uint32_t q = mant >> shift;
        const uint32_t rest = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        q += (rest > halfway || (rest == halfway && (q & 1u))) ? 1u : 0u;
        return static_cast<uint16_t>(sign | q);
    }
    uint32_t q = sign | (static_cast<uint32_t>(e) << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    q += (rest > 0x1000u || (rest == 0x1000u && (q & 1u))) ? 1u : 0u;
    return static_cast<uint16_t>(q);
}

// Exact float value of an IEEE binary16 pattern (common.h:33-55 semantics).
float from_half_bits(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu, bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e > 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        int lz = 0;
        while (!(m & 0x400u)) {
            m <<= 1;
            lz++;
        }
        bits = sign | (static_cast<uint32_t>(113 - lz) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = static_cast<uint8_t>(v);
    p[1] = static_cast<uint8_t>(v >> 8);
}

float block_max_abs(const float* x) {
    float m = 0.0f;
    for (int i = 0; i < kBlock; i++) m = std::max(m, std::fabs(x[i]));  // NaN never wins
    return m;
}

// E4M3 by rounding the f16 pattern of y/256 at bit 7 (quant.cpp:43-49).
uint8_t fp8_code(float y) {
    const uint16_t h = to_half_bits(y * (1.0f / 256.0f));
    const uint32_t mag = h & 0x7fffu;
    const uint32_t c = std::min<uint32_t>((mag + 0x3fu + ((mag >> 7) & 1u)) >> 7, 0x7eu);
    return static_cast<uint8_t>(c | ((h >> 8) & 0x80u));
}

// E2M1 by thresholds halfway between the magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6} (quant.cpp:57-61).
uint8_t fp4_code(float y) {
    static const float kEdges[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    const float a = std::fabs(y);
    int c = 0;
    for (float edge : kEdges) c += a > edge ? 1 : 0;
    return static_cast<uint8_t>(c == 0 ? 0 : (c | (y < 0 ? 8 : 0)));
}

float fp4_nearest(float a) {  // quant.cpp:93-97
    if (a < 1.75f) return std::nearbyint(a * 2.0f) * 0.5f;
    if (a < 3.5f) return std::nearbyint(a);
    return a < 5.0f ? 4.0f : 6.0f;
}

struct Fit {
    float err, xr, rr;
};

// Squared error of the block at scale s plus the least-squares sums, sequential float sums
// (quant.cpp:126-137).
Fit fp4_fit(const float* ax, float s) {
    Fit f{0.0f, 0.0f, 0.0f};
    const float inv = 1.0f / s;
    for (int i = 0; i < kBlock; i++) {
        const float r = fp4_nearest(ax[i] * inv);
        const float d = ax[i] - r * s;
        f.err += d * d;
        f.xr += ax[i] * r;
        f.rr += r * r;
    }
    return f;
}

// amax/6 then up to two refits while the squared error keeps dropping (quant.cpp:142-165).
uint16_t fp4_scale(const float* xb) {
    uint16_t best = to_half_bits(block_max_abs(xb) / 6.0f);
    if (from_half_bits(best) <= 0) return 0;
    float ax[kBlock];
    for (int i = 0; i < kBlock; i++) ax[i] = std::fabs(xb[i]);
    Fit fit = fp4_fit(ax, from_half_bits(best));
    float best_err = fit.err;
    for (int round = 0; round < 2 && fit.rr > 0; round++) {
        const uint16_t s = to_half_bits(fit.xr / fit.rr);
        if (from_half_bits(s) <= 0 || s == best) break;
        fit = fp4_fit(ax, from_half_bits(s));
        if (fit.err >= best_err) break;
        best_err = fit.err;
        best = s;
    }
    return best;
}

void encode_row(int fmt, const float* x, int64_t cols, uint8_t* out) {
    if (fmt == NEKO_FMT_F16) {
        for (int64_t c = 0; c < cols; c++) put16(out + 2 * c, to_half_bits(x[c]));
        return;
    }
    const int64_t nb = cols / kBlock;
    uint8_t* scales = out + (fmt == NEKO_FMT_FP8 ? cols : cols / 2);
    for (int64_t b = 0; b < nb; b++) {
        const float* xb = x + b * kBlock;
        if (fmt == NEKO_FMT_FP8) {  // quant.cpp:72-90
            const uint16_t s = to_half_bits(block_max_abs(xb) / 448.0f);
            const float sv = from_half_bits(s);
            const float inv = sv > 0 ? 1.0f / sv : 0.0f;
            put16(scales + 2 * b, sv > 0 ? s : 0);
            for (int i = 0; i < kBlock; i++) out[b * kBlock + i] = fp8_code(xb[i] * inv);
        } else {  // quant.cpp:167-178
            const uint16_t s = fp4_scale(xb);
            put16(scales + 2 * b, s);
            const float inv = s ? 1.0f / from_half_bits(s) : 0.0f;
            uint8_t* o = out + b * (kBlock / 2);
            for (int j = 0; j < kBlock / 2; j++)
                o[j] = static_cast<uint8_t>(fp4_code(xb[j] * inv) | (fp4_code(xb[kBlock / 2 + j] * inv) << 4));
        }
    }
}

}  // namespace

extern "C" {

size_t neko_quant_row_bytes(int fmt, int64_t cols) {
    if (cols < 0) return 0;
    const size_t c = static_cast<size_t>(cols);
    const size_t scale_bytes = (c / kBlock * 2 + 15) / 16 * 16;
    switch (fmt) {
        case NEKO_FMT_F16: return 2 * c;
        case NEKO_FMT_FP8: return c + scale_bytes;
        case NEKO_FMT_FP4: return c / 2 + scale_bytes;
    }
    return 0;
}

int neko_quantize_rows(int fmt, int64_t rows, int64_t cols, const float* src, uint8_t* dst, int threads, int* fmt_used) {
    if (fmt != NEKO_FMT_F16 && fmt != NEKO_FMT_FP8 && fmt != NEKO_FMT_FP4) return NEKO_ERR_INVALID;
    if (rows < 0 || cols <= 0) return NEKO_ERR_INVALID;
    if (cols % kBlock != 0) fmt = NEKO_FMT_F16;  // quant.cpp:257
    if (fmt_used) *fmt_used = fmt;
    if (rows == 0) return NEKO_OK;
    if (!src || !dst) return NEKO_ERR_INVALID;
    const size_t rb = neko_quant_row_bytes(fmt, cols);
    int n = threads > 0 ? threads : static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
    n = static_cast<int>(std::min<int64_t>(n, rows));
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++) {
            uint8_t* out = dst + static_cast<size_t>(r) * rb;
            std::memset(out, 0, rb);  // scale padding is zero
            encode_row(fmt, src + r * cols, cols, out);
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n; i++) pool.emplace_back(work, rows * i / n, rows * (i + 1) / n);
    work(0, rows / n);
    for (auto& t : pool) t.join();
    return NEKO_OK;
}

int neko_rope_table(double theta, int hd, int64_t n_pos, float* cs) {
    if (hd <= 0 || hd % 2 != 0 || n_pos < 0) return NEKO_ERR_INVALID;
    if (n_pos == 0) return NEKO_OK;
    if (!cs) return NEKO_ERR_INVALID;
    for (int i = 0; i < hd / 2; i++) {
        const double inv_freq = std::pow(theta, -2.0 * i / hd);
        for (int64_t p = 0; p < n_pos; p++) {
            const double angle = static_cast<double>(p) * inv_freq;
            float* pair = cs + p * hd + 2 * i;
            pair[0] = static_cast<float>(std::cos(angle));
            pair[1] = static_cast<float>(std::sin(angle));
        }
    }
    return NEKO_OK;
}

}  // extern "C"
