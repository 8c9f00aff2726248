// E2M1 (FP4) and E4M3 (FP8) codes from gfx950's conversion instructions, corrected to equal the
// reference quantiser's own arithmetic (quant.cpp) on every input. Shared by the device quantiser and
// tests/cpp/quant_codes_check.hip, which compares each against that arithmetic over every f32 bit
// pattern on the GPU.
#pragma once

#include "device.h"

namespace neko_hip {

typedef short short2v __attribute__((ext_vector_type(2)));

// quant.cpp:43-49 for four values, packed little-endian: the f16 pattern of y/256, rounded to nearest
// even over its 7 low bits, clamped to 0x7E (448; 0x7F would decode as 480). Those bits are the E4M3
// code of 256 x f16(y/256): the hardware conversion of f16 to E4M3 with scale 1/256 (round to nearest
// even) gives the same byte for every f16 whose magnitude times 256 stays below 452; past that it
// returns the NaN code where the reference clamps to 448, so y is clamped to +-448 first (its codes
// there are 0x7E / 0xFE either way). f16(y/256) is the reference's own rounding, kept as a separate
// step: the double rounding is part of its result. Equal to the reference for every non-NaN y.
__device__ __forceinline__ uint32_t encode_fp8x4(float y0, float y1, float y2, float y3) {
    const auto h = [](float y) { return f16_rne(__builtin_amdgcn_fmed3f(y, -448.0f, 448.0f) * (1.0f / 256.0f)); };
    const short2v lo = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(short2v{0, 0}, half2v{h(y0), h(y1)}, 1.0f / 256.0f, false);
    const short2v both = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(lo, half2v{h(y2), h(y3)}, 1.0f / 256.0f, true);
    return __builtin_bit_cast(uint32_t, both);
}

// quant.cpp:57-61 encodes |y| by a threshold ladder: the nearest E2M1 magnitude with every tie
// (0.25, 0.75, ..., 5.0) rounded down, the sign kept only on a nonzero magnitude, and NaN as 0. The
// hardware conversion (round to nearest even) differs only at the ties it rounds up -- 0.75, 1.75,
// 3.5 -- and in the sign of a zero magnitude, so those inputs are replaced first (a tie by a value
// below it, |y| <= 0.25 or NaN by +0); with that, code = ladder for every f32 pattern. Returns the
// input to hand the conversion.
__device__ __forceinline__ float fp4_encode_input(float y) {
    const float a = fabsf(y);
    const bool tie_up = a == 0.75f || a == 1.75f || a == 3.5f;
    return !(a > 0.25f) ? 0.0f : (tie_up ? y * 0.9f : y);
}

// quant.cpp:93-97: nearest E2M1 magnitude of a >= 0, for two values at once. The hardware E2M1
// conversion (round to nearest even; NaN and values past 6 give 6) returns the reference's
// threshold ladder's value for every non-negative f32 but 5.0, the one tie the ladder rounds up (to 6)
// where nearest-even rounds down (to 4). One conversion each way for the pair, and the 5.0 case set
// explicitly, in place of the ladder's two roundings and three selects per value.
__device__ __forceinline__ float2v fp4_round2(float a0, float a1) {
    const uint32_t code = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, a0, a1, 1.0f, 0);
    float2v r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(code, 1.0f, 0);
    r.x = a0 == 5.0f ? 6.0f : r.x;
    r.y = a1 == 5.0f ? 6.0f : r.y;
    return r;
}

}  // namespace neko_hip
