// Shared helpers of libmamba_int: status reporting, argument checks and the
// integer rounding/saturation primitives of spec mi-spec-2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "mamba_int.h"

namespace mi {

// Records a message for mi_last_error_string() and returns `st`.
mi_status fail(mi_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks the launch just enqueued; returns MI_OK or MI_ERR_HIP with a message.
mi_status check_launch(const char *what);
// Clears the calling thread's error message (start of every entry point).
void clear_error();

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Compute units of the current device (cached per device; 256 if the query fails).
inline int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// The wave index within the block as a scalar, so the compiler treats
// branches on it as uniform (no per-lane masking around loads).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Sums over the 4 lanes of a quad by DPP quad swaps (quad_perm [1,0,3,2],
// then [2,3,0,1]), with no LDS round trip; every lane of the quad must be
// active.
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    return v;
}
template <int kCtrl>
__device__ __forceinline__ int64_t dpp_add64(int64_t v) {
    const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)v, kCtrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)((uint64_t)v >> 32), kCtrl, 0xF, 0xF, false);
    return v + (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int64_t quad_sum64(int64_t v) { return dpp_add64<0x4E>(dpp_add64<0xB1>(v)); }

// ------------------------------------------------------ integer primitives
__host__ __device__ __forceinline__ constexpr int64_t rshr64(int64_t v, int s) {
    return s <= 0 ? v : ((v + ((int64_t)1 << (s - 1))) >> s);
}
__host__ __device__ __forceinline__ int32_t rshr32(int32_t v, int s) {
    // exact for |v| < 2^31 - 2^(s-1): callers guarantee it (|acc| <= K*127)
    return s <= 0 ? v : ((v + (1 << (s - 1))) >> s);
}
__host__ __device__ __forceinline__ int32_t clamp32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
__host__ __device__ __forceinline__ constexpr int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
__host__ __device__ __forceinline__ int32_t sat32_64(int64_t v) {
    return (int32_t)clamp64(v, INT32_MIN, INT32_MAX);
}
__host__ __device__ __forceinline__ int32_t sat8(int32_t v) { return clamp32(v, -127, 127); }
constexpr int32_t kResidualLimit = (1 << 23) - 1;

// One step of the dyadic recurrence at decay shift 15, for one state:
// h <- sat32(floor(h * n / 2^15) + u), and the state's two exact y partials.
// h is read as two 16-bit fields, H = h >> 16 (signed) and L = h & 0xffff,
// with n2 = 2n <= 2^16:  floor(h*n/2^15) = H*n2 + floor(L*n2/2^16), exactly
// (H*n2 is an integer), with L*n2 < 2^32 and |H*n2| <= 2^31.  y = C . h is
// kept as yhi = sum C*H and ylo = sum C*L (y = yhi * 2^16 + ylo; both stay in
// int32 for up to 128 states of int8 C).  The fields are word halves, so the
// 24-bit multiplies read them through SDWA operand selects: the update is
// three multiplies, an add and the clamped add, and y two multiplies and
// their share of the adds.
__device__ __forceinline__ void update16(int32_t &h, int n2, int u, int cv, int &yhi, int &ylo) {
    // The products are kept as plain multiplies (the empty asm hides them from
    // mad formation): fused into a v_mad_i32_i24, H or L would need a shift or
    // a mask of its own, where v_mul_*_u24/i24 read them as SDWA word selects.
    int dh = __mul24(h >> 16, n2);
    asm("" : "+v"(dh));
    const uint32_t cl = __umul24((uint32_t)h & 0xffffu, (uint32_t)n2);
    h = __builtin_elementwise_add_sat(dh + (int)(cl >> 16), u);
    int ph = __mul24(cv, h >> 16), pl = __mul24(cv, h & 0xffff);
    asm("" : "+v"(ph), "+v"(pl));
    yhi += ph;
    ylo += pl;
}

typedef short mi_short2 __attribute__((ext_vector_type(2)));

// sat32(b * x + d) for b, x in 24-bit signed range: v_mad_i32_i24 with the
// clamp bit saturates the full-precision sum (checked on the hardware against
// a 64-bit saturating reference, both directions)
__device__ __forceinline__ int mad24_sat(int b, int x, int d) {
    int r;
    asm("v_mad_i32_i24 %0, %1, %2, %3 clamp" : "=v"(r) : "v"(b), "v"(x), "v"(d));
    return r;
}

// update16 with the input term as the pair (b, x), u = b * x: the input and
// the saturating add are one clamped v_mad_i32_i24
__device__ __forceinline__ void update16_b(int32_t &h, int n2, int b, int x, int cv, int &yhi, int &ylo) {
    int dh = __mul24(h >> 16, n2);
    asm("" : "+v"(dh));
    const uint32_t cl = __umul24((uint32_t)h & 0xffffu, (uint32_t)n2);
    h = mad24_sat(b, x, dh + (int)(cl >> 16));
    // (no barrier on the y products here: behind the clamped multiply-add the
    // compiler keeps them as SDWA multiplies by itself, and an asm statement
    // costs an s_nop after it)
    yhi += __mul24(cv, h >> 16);
    ylo += __mul24(cv, h & 0xffff);
}

// update16 for a coefficient held as cs = C * 2^16 (C in the high half, zero
// low half) and the input term as the pair (b, x), u = b * x: the input and
// the saturating add are one clamped v_mad_i32_i24; yhi accumulates H*C in one
// v_dot2c_i32_i16 on the state's two halves (the low half meets the zero), and
// ylo reads C as cs's high word.
__device__ __forceinline__ void update16_cs(int32_t &h, int n2, int b, int x, int cs, int &yhi, int &ylo) {
    int dh = __mul24(h >> 16, n2);
    asm("" : "+v"(dh));
    const uint32_t cl = __umul24((uint32_t)h & 0xffffu, (uint32_t)n2);
    h = mad24_sat(b, x, dh + (int)(cl >> 16));
    yhi = __builtin_amdgcn_sdot2(__builtin_bit_cast(mi_short2, h), __builtin_bit_cast(mi_short2, cs), yhi, false);
    int pl = __mul24(cs >> 16, h & 0xffff);
    asm("" : "+v"(pl));
    ylo += pl;
}

// update16_cs for a lane's first state: its products start y's two partial
// sums (yhi = C*H, ylo = C*L, one word-select multiply each) instead of
// accumulating onto zeroed sums
__device__ __forceinline__ void update16_cs_first(int32_t &h, int n2, int b, int x, int cs, int &yhi, int &ylo) {
    int dh = __mul24(h >> 16, n2);
    asm("" : "+v"(dh));
    const uint32_t cl = __umul24((uint32_t)h & 0xffffu, (uint32_t)n2);
    h = mad24_sat(b, x, dh + (int)(cl >> 16));
    // (kept out of mad formation: a v_mad_i32_i24 with the first DPP stage
    // would need H and L shifted and masked out first)
    yhi = __mul24(cs >> 16, h >> 16);
    ylo = __mul24(cs >> 16, h & 0xffff);
    asm("" : "+v"(yhi), "+v"(ylo));
}

// Exact floor(sqrt(v)) for v < 2^62 (host and device): a float estimate
// refined by integer correction steps.
__host__ __device__ __forceinline__ uint64_t isqrt64(uint64_t v) {
    uint64_t s = (uint64_t)sqrt((double)v);
    while (s * s > v) --s;
    while ((s + 1) * (s + 1) <= v) ++s;
    return s;
}

// BitShiftNorm parameters of one row (spec rule 4.1) from its exact row
// statistics s1 = sum r, s2 = sum r^2: mu = floor(s1/dim) and
// S = sum (r - mu)^2 = s2 - 2 mu s1 + dim mu^2 (exact in int64 for
// |r| < 2^23, dim <= 8192); returns the output shift 12 + k of the threshold
// table (mamba_integer_model.py:169-182 on var = S / (dim * 2^16)).
// KMAX / KMIN: the table's count of "var >= 4^j" and "var < 4^-j" steps.
template <int KMAX, int KMIN>
__host__ __device__ __forceinline__ int norm_shift_tab(int64_t s1, int64_t s2, int dim, int64_t *mu_out) {
    // floor(s1 / dim) through one double division: |s1| < 2^36 (|r| < 2^23,
    // dim <= 8192), so the rounded quotient is within 2^-17 of the exact one,
    // which is an integer or at least 1/dim >= 2^-13 away from one; the floor
    // is exact (and far shorter on the GPU than a 64-bit integer division)
    const int64_t mu = (int64_t)floor((double)s1 / (double)dim);
    const int64_t S = s2 - 2 * mu * s1 + (int64_t)dim * mu * mu;
    int kk = 0;
    for (int j = 1; j <= KMAX; ++j) kk += S >= ((int64_t)dim << (2 * (j + 8)));
    for (int j = 1; j <= KMIN; ++j) kk -= S < ((int64_t)dim << (2 * (8 - j)));
    *mu_out = mu;
    return 12 + kk;
}
__host__ __device__ __forceinline__ int norm_shift(int64_t s1, int64_t s2, int dim, int64_t *mu_out) {
    return norm_shift_tab<8, 3>(s1, s2, dim, mu_out);
}
// BitShiftNormV2's table (ssd_multihead.py:613-629; spec rule 7.1): scales
// 2^-1 .. 2^-6 for var >= 4 .. 4096, 2 and 4 for var < 1/4 and < 1/16.
template <bool V2>
__host__ __device__ __forceinline__ int norm_shift_for(int64_t s1, int64_t s2, int dim, int64_t *mu_out) {
    return V2 ? norm_shift_tab<6, 2>(s1, s2, dim, mu_out) : norm_shift_tab<8, 3>(s1, s2, dim, mu_out);
}

// dt of spec rule 4.8 (mamba_integer_model.py:427) for dm in [-20, 20].
__host__ __device__ inline int32_t dt_q16(int dm) {
    int64_t s = (int64_t)dm * 65536 +
                (int64_t)isqrt64((uint64_t)((int64_t)dm * dm) * (1ull << 32) + (1ull << 34));
    int64_t sq = s >> 1;
    return (int32_t)clamp64(rshr64(655 * sq, 16), 66, 6554);
}

// floor(sqrt(v)) digit by digit, for tables built at compile time.
constexpr uint64_t isqrt64_bitwise(uint64_t v) {
    uint64_t r = 0, bit = 1ull << 62;
    while (bit > v) bit >>= 2;
    while (bit) {
        if (v >= r + bit) {
            v -= r + bit;
            r = (r >> 1) + bit;
        } else {
            r >>= 1;
        }
        bit >>= 2;
    }
    return r;
}

// dt_q16 in a constant expression (same rule, bitwise square root).
constexpr int32_t dt_q16_table_entry(int dm) {
    const int64_t s = (int64_t)dm * 65536 + (int64_t)isqrt64_bitwise((uint64_t)((int64_t)dm * dm) * (1ull << 32) +
                                                                     (1ull << 34));
    return (int32_t)clamp64(rshr64(655 * (s >> 1), 16), 66, 6554);
}

// Gate of spec rule 4.11 (mamba_integer_model.py:124-132), Q15, z in Q4.
__host__ __device__ constexpr int32_t gate_q15(int z) {
    int32_t a = z < 0 ? -z : z;
    int32_t q = (16384 * a) / (16 + a);
    return 16384 + (z < 0 ? -q : q);
}

// The decode step kernels' lookup tables, built by the compiler: dt_q16(dm)
// for dm in [-20, 20] and gate_q15(z) for z in [-128, 127].  Blocks copy
// them into LDS with one load per thread instead of evaluating the rules.
struct StepTables {
    int32_t dtq[41];
    int32_t gate[256];
};
constexpr StepTables make_step_tables() {
    StepTables t{};
    for (int i = 0; i < 41; ++i) t.dtq[i] = dt_q16_table_entry(i - 20);
    for (int i = 0; i < 256; ++i) t.gate[i] = gate_q15(i - 128);
    return t;
}
// Position-weighted sums of both tables as the integer oracle computes them
// (sum (i + 1) * table[i]), so a wrong entry fails the build.
constexpr int64_t step_table_weighted_sum(const int32_t *t, int n) {
    int64_t s = 0;
    for (int i = 0; i < n; ++i) s += (int64_t)(i + 1) * t[i];
    return s;
}
static_assert(step_table_weighted_sum(make_step_tables().dtq, 41) == 3482397, "dt table");
static_assert(step_table_weighted_sum(make_step_tables().gate, 256) == 756841947, "gate table");

}  // namespace mi

#define MI_REQUIRE(cond, st, ...)                     \
    do {                                              \
        if (!(cond)) return ::mi::fail((st), __VA_ARGS__); \
    } while (0)
