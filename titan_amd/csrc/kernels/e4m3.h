// e4m3.h -- FP8 E4M3 quantisation shared by the append kernels and the fused
// decode-step append (OCP E4M3FN: bias 7, S.1111.111 = NaN, max 448), so that
// every path stores the same code for the same value.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Round to nearest, ties to even mantissa; |x| >= 448 (and inf) saturates to
// +-448; NaN -> S.1111.111.
__device__ __forceinline__ uint32_t e4m3_code(float y) {
    const uint32_t u = __float_as_uint(y);
    const uint32_t s = (u >> 24) & 0x80u;
    const float a = __builtin_fabsf(y);
    if (a != a) return s | 0x7Fu;
    if (a >= 448.0f) return s | 0x7Eu;
    if (a < 0.015625f) return s | (uint32_t)__builtin_rintf(a * 512.0f);  // 2^-9 grid; 8 = 2^-6
    int e = (int)((u >> 23) & 0xFFu) - 127;                               // a in [2^e, 2^(e+1))
    const float mant = __uint_as_float((u & 0x007FFFFFu) | 0x3F800000u);   // a / 2^e in [1, 2)
    uint32_t m = (uint32_t)__builtin_rintf(mant * 8.0f) - 8u;             // 0..8
    if (m == 8u) { ++e; m = 0u; }
    const uint32_t code = ((uint32_t)(e + 7) << 3) | m;
    return s | (code < 0x7Eu ? code : 0x7Eu);
}
