// Test-only: the quantiser's hardware-conversion codes (nekochat_amd/csrc/quant_codes.h) against the
// reference quantiser's own arithmetic, restated here as the check, over every f32 bit pattern.
// Output: _build/libquant_codes_check.so (loaded by tests/test_gpu_quant_codes.py).
#include "../../nekochat_amd/csrc/quant_codes.h"

namespace {

using namespace neko_hip;

// quant.cpp:93-97 fp4 rounding of a >= 0: the threshold ladder.
__device__ float ref_fp4_round(float a) {
    if (a < 1.75f) return __builtin_rintf(a * 2.0f) * 0.5f;
    if (a < 3.5f) return __builtin_rintf(a);
    return a < 5.0f ? 4.0f : 6.0f;
}

// quant.cpp:57-61 fp4 encode: magnitude = thresholds strictly below |y|; sign only on nonzero codes.
__device__ uint32_t ref_encode_fp4(float y) {
    const float a = fabsf(y);
    const uint32_t c = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.0f);
    return c == 0 ? 0u : (c | (y < 0.0f ? 8u : 0u));
}

// quant.cpp:43-49 fp8 encode: halfBits(y / 256) (one RNE f32 -> f16 conversion), rounded to nearest
// even over its 7 low bits, clamped to 0x7E, with the f16 sign.
__device__ uint32_t ref_encode_fp8(float y) {
    const uint32_t h = __builtin_bit_cast(uint16_t, f16_rne(y * (1.0f / 256.0f)));
    const uint32_t mag = h & 0x7FFFu;
    uint32_t c = (mag + 0x3Fu + ((mag >> 7) & 1u)) >> 7;
    if (c > 0x7Eu) c = 0x7Eu;
    return c | ((h >> 8) & 0x80u);
}

constexpr int kPer = 64;  // patterns per thread

// which 0: fp4_round2 over the 2^31 non-negative patterns; 1: the fp4 encode over all 2^32; 2: the
// fp8 encode over all 2^32. counts[2 * which + (pattern is NaN)] += mismatches; first[which] = the
// lowest mismatching pattern.
__global__ void check_kernel(int which, uint64_t n, unsigned long long* counts, uint32_t* first) {
    const uint64_t base = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * kPer;
    for (int i = 0; i < kPer; i++) {
        const uint64_t u = base + i;
        if (u >= n) return;
        const uint32_t bits = static_cast<uint32_t>(u);
        const float y = __builtin_bit_cast(float, bits);
        bool bad;
        if (which == 0) {
            const float2v r = fp4_round2(y, y);
            const uint32_t want = __builtin_bit_cast(uint32_t, ref_fp4_round(y));
            bad = __builtin_bit_cast(uint32_t, r.x) != want || __builtin_bit_cast(uint32_t, r.y) != want;
        } else if (which == 1) {
            const uint32_t byte = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, fp4_encode_input(y), fp4_encode_input(y), 1.0f, 0);
            const uint32_t want = ref_encode_fp4(y);
            bad = (byte & 0xFFu) != (want | (want << 4));
        } else {
            const uint32_t word = encode_fp8x4(y, y, y, y);
            const uint32_t want = ref_encode_fp8(y);
            bad = word != want * 0x01010101u;
        }
        if (bad) {
            const bool nan = (bits & 0x7FFFFFFFu) > 0x7F800000u;
            atomicAdd(&counts[2 * which + (nan ? 1 : 0)], 1ull);
            atomicMin(&first[which], bits);
        }
    }
}

}  // namespace

// counts[6], first[3]; returns 0 or the HIP error code.
extern "C" int neko_test_quant_codes(unsigned long long* counts, uint32_t* first) {
    unsigned long long* d_counts = nullptr;
    uint32_t* d_first = nullptr;
    hipError_t e = hipMalloc(&d_counts, 6 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc(&d_first, 3 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(d_counts, 0, 6 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemset(d_first, 0xFF, 3 * sizeof(uint32_t));
    for (int which = 0; which < 3 && e == hipSuccess; which++) {
        const uint64_t n = which == 0 ? (1ull << 31) : (1ull << 32);
        const uint32_t blocks = static_cast<uint32_t>(n / (256ull * kPer));
        hipLaunchKernelGGL(check_kernel, dim3(blocks), dim3(256), 0, 0, which, n, d_counts, d_first);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(counts, d_counts, 6 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(first, d_first, 3 * sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (d_counts) (void)hipFree(d_counts);
    if (d_first) (void)hipFree(d_first);
    return static_cast<int>(e);
}
