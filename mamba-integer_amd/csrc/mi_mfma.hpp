// Ternary unpack and the int8 MFMA used by every BitLinear kernel.
#pragma once

#include "mi_common.hpp"

namespace mi {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef long long v2l __attribute__((ext_vector_type(2)));  // (sum r, sum r^2) pairs

// 16 ternary weights of one packed word -> 16 int8 in k order (4 dwords).
// (word >> 2j) & 0x03030303 holds the 2-bit codes of weights 4j..4j+3 in byte
// order; v_perm_b32 against the byte table {0x00, 0x01, 0xFE, 0xFF} (byte c =
// value of code c, both permute sources equal) sign-extends all four at once.
__device__ __forceinline__ v4i unpack16(uint32_t w) {
    const uint32_t lut = 0xFFFE0100u;
    v4i r;
    r[0] = (int)__builtin_amdgcn_perm(lut, lut, w & 0x03030303u);
    r[1] = (int)__builtin_amdgcn_perm(lut, lut, (w >> 2) & 0x03030303u);
    r[2] = (int)__builtin_amdgcn_perm(lut, lut, (w >> 4) & 0x03030303u);
    r[3] = (int)__builtin_amdgcn_perm(lut, lut, (w >> 6) & 0x03030303u);
    return r;
}

// D(16x16) += A(16x64) * B(64x16), int8 in, int32 accumulate (gfx950).
__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Exact squareplus of spec rule 4.4 on a conv output c (Q10) -> int8 (Q4):
// floor(sqrt(v^2 + 2^22)) from the hardware square root of the float-rounded
// argument.  With 2^22 <= Y < 2^32, rounding Y to float moves sqrt(Y) by at
// most 128 / (2 * 2048) < 0.032 and v_sqrt_f32 adds under an ulp (2^-8), so
// the truncated root is isqrt(Y) or one off; one compare each way makes it
// exact (s <= 51243, so the 24-bit squares are exact).
__device__ __forceinline__ int sqp_q(int32_t c) {
    const int32_t v = clamp32(c, -51200, 51200);
    const uint32_t av = (uint32_t)(v < 0 ? -v : v);
    const uint32_t Y = __umul24(av, av) + (1u << 22);  // av <= 51200: the 24-bit product is exact, < 2^32
    uint32_t s = (uint32_t)__builtin_amdgcn_sqrtf((float)Y);
    s -= __umul24(s, s) > Y ? 1u : 0u;
    s += __umul24(s + 1, s + 1) <= Y ? 1u : 0u;
    return clamp32(rshr32(v + (int32_t)s, 7), -127, 127);
}

}  // namespace mi
