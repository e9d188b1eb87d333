// mx_encode.h -- the element encoders of the MX quantizers: E2M1 for MXFP4
// (python/quantize_mxfp4.py:18-39) and E4M3 for the MX-FP8 activation format,
// shared by the gfx950 quantize kernels and a host test that checks them
// against the oracle for every float a block can produce.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define MX4_HOST_DEVICE __host__ __device__ __forceinline__
#else
#define MX4_HOST_DEVICE inline
#endif

namespace mx4 {

// Code (0..7) of a magnitude already divided by its block's scale, for
// 0 <= scaled <= 8 (the scale rule keeps every value of a block below 8):
// the nearest of the levels {0, 1/2, 1, 3/2, 2, 3, 4, 6}, ties to the even
// code, 6 above 5. Below 1 the levels are the multiples of 1/2, so the code
// is rint(2 scaled) (round half to even). From 1 on a level is 1.m x 2^e with
// one mantissa bit: rounding the float's 23-bit mantissa to its top bit, half
// to even, then reading exponent and that bit gives code 2 + 2e + m; a carry
// out of [4, 8) lands on 8 and saturates to code 7 (6).
MX4_HOST_DEVICE uint32_t e2m1_magnitude_code(float scaled) {
    const uint32_t sub = (uint32_t)__builtin_rintf(scaled * 2.0f);
    const uint32_t b = __builtin_bit_cast(uint32_t, scaled);
    const uint32_t r = b + 0x1FFFFFu + ((b >> 22) & 1u);
    uint32_t c = 2u * ((r >> 23) - 127u) + 2u + ((r >> 22) & 1u);
    c = c > 7u ? 7u : c;
    return scaled < 1.0f ? sub : c;
}

// E4M3 code (0..0x7e) of a magnitude already divided by its block's scale,
// for 0 <= scaled < 512 (the MX-FP8 scale rule keeps a block below 512): the
// nearest E4M3 value, ties to the even code, 448 (0x7e) above it. Below 2^-6
// the values are the multiples of 2^-9, so the code is rint(512 scaled); from
// 2^-6 on the float's mantissa is rounded to its top 3 bits, half to even, and
// the code is (e + 7) << 3 | m, saturated at 0x7e.
MX4_HOST_DEVICE uint32_t e4m3_magnitude_code(float scaled) {
    const uint32_t sub = (uint32_t)__builtin_rintf(scaled * 512.0f);
    const uint32_t b = __builtin_bit_cast(uint32_t, scaled);
    const uint32_t r = b + 0x7FFFFu + ((b >> 20) & 1u);
    uint32_t c = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);  // (e + 7) << 3 with e = exponent - 127
    c = c > 0x7eu ? 0x7eu : c;
    return scaled < 0.015625f ? sub : c;
}

}  // namespace mx4
