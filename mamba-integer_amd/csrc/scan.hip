// Dyadic selective scans for gfx950 (spec mi-spec-2, rule 1 and 4.7-4.11).
//
// The recurrence h_t = sat32(floor(h_{t-1} * n / 2^k) + u_t) is not
// associative (the floor does not compose), so exact parallelism comes only
// from independent lanes: (batch, head, channel, state).  Time stays
// sequential inside every lane.  The scan is integer-VALU bound, so the
// kernels are built around a short per-update instruction sequence:
//
//   the state h is read as two 16-bit fields, H = h >> 16 (signed) and
//   L = h & 0xffff, with n2 = 2n = n * 2^(16-k) <= 2^16:
//     d   = H * n2 + ((L * n2) >> 16)    v_mul_i32_i24, v_mul_u32_u24, v_add_u32
//     h'  = sat32(d + B * x)             v_mad_i32_i24 clamp (S >= 4; else
//                                        an SDWA multiply and v_add_i32 clamp)
//     yhi += C*H'; ylo += C*L'           2 x v_mul_i32_i24 + adds  (exact int32 partials)
//
// floor(h*n/2^15) = H*n2 + floor(L*n2/2^16) exactly because H*n2 is an
// integer (h*n/2^15 = h*n2/2^16), and y = 2^16 * sum(C*H) + sum(C*L) is
// recombined in int64 once per step.  The fields are word halves, so every
// read of H and L is an SDWA operand select: no shift or mask per state.
// This holds for 0 <= n <= 2^k with k = 15 and N <= 128 (L*n2 < 2^32,
// |H*n2| <= 2^31, |sum C*H| <= 128*128*2^15 = 2^29, |sum C*L| < 2^31); other
// shifts and shapes take the plain int64 kernels at the end.
//
// Layout: a block owns CH = 256/G channels of one (batch, head); G adjacent
// lanes share a channel and hold S = N/G states each; their partial y sums
// are combined with DPP adds.  Inputs of TC time steps are staged through LDS
// (prefetched into registers one chunk ahead), x bytes transposed to
// channel-major so one ds_read_b32 serves 4 steps, B widened to int32 for the
// clamped multiply-add where a lane holds four or more states; outputs are
// staged in LDS and written with 16-byte stores.
#include <type_traits>

#include "mi_common.hpp"

namespace mi {
namespace {

constexpr int kThreads = 256;
constexpr int kTC = 64;  // time steps per staged chunk

enum ScanMode { kModeChannel = 0, kModeHead = 1, kModeModel = 2 };

template <int G>
__device__ __forceinline__ int group_sum(int v) {
    // Sum over the G adjacent lanes of a channel group; every lane gets it.
    if constexpr (G >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    if constexpr (G >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    if constexpr (G >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    if constexpr (G >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); // row_mirror
    return v;
}

__device__ __forceinline__ int sbyte(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }

struct ScanArgs {
    const int8_t *x;       // channel/head modes: x; model mode: xs
    const int8_t *bsrc;    // B rows
    const int8_t *csrc;    // C rows
    const int32_t *decay;  // [P][N] (channel), [H] (head), base [P][N] (model)
    int32_t *y;            // int32 y (channel/head)
    int8_t *yo;            // int8 gated output (model)
    int32_t *chunk_states; // head mode, nullable
    const int32_t *h_in;
    int32_t *h_out;
    const int8_t *dm;      // model
    const int8_t *z;       // model
    int64_t x_row;         // element stride between consecutive (b,t) rows of x/y (= H*P)
    int64_t bc_row;        // stride between consecutive (b,t) rows of B/C
    int64_t z_row;         // model: row stride of z
    int B, L, H, P;
    int k;
    int s_y;
    int nchunks_out;       // head mode: number of chunk_states chunks (ceil(L/cs))
    int cs;                // head mode: chunk length of chunk_states
};

// Loads 16 consecutive bytes (16-byte aligned) or zeros when out of range.
__device__ __forceinline__ uint4 load16(const int8_t *p, bool ok) {
    if (ok) return *reinterpret_cast<const uint4 *>(p);
    return make_uint4(0, 0, 0, 0);
}

template <int N, int G, int MODE>
__global__ __launch_bounds__(kThreads) void scan_kernel(ScanArgs a) {
    static_assert(MODE != kModeModel, "the fused model scan has its own kernel (model_scan.hip)");
    constexpr int S = N / G;
    constexpr int CH = kThreads / G;
    constexpr int XP = kTC + 4;                 // padded row of the transposed x tile
    constexpr int X16 = CH / 16;                // 16-byte pieces per time row of x
    constexpr int XPIECES = kTC * X16;          // per chunk
    constexpr int XPER = (XPIECES + kThreads - 1) / kThreads;
    constexpr int BC16 = N / 16;
    constexpr int BCPIECES = kTC * BC16;
    constexpr int BCPER = (BCPIECES + kThreads - 1) / kThreads;

    __shared__ __align__(16) int8_t s_x[CH][XP];
    // WIDEB: B widened to int32, so the input term B * x and the saturating
    // add are one clamped v_mad_i32_i24 (which takes no SDWA byte select).
    // Lanes of one or two states keep B as bytes: their latency-bound chain
    // measured slower with the wider staging (config 1: 22.0 -> 25.1 us)
    constexpr bool WIDEB = S >= 4;
    constexpr bool STAGE_Y = CH <= 64;  // int32 y staged in LDS (16 KB at most)
    // blocks of <= 32 channels (G >= 8) reduce the y partials of four steps
    // together and park the exact (yhi, ylo) pairs here; the chunk epilogue
    // recombines and saturates once per (step, channel)
    constexpr bool DEFER = CH <= 32;
    // C32: C staged as int32 C * 2^16 as well (update16_cs: y's high partial
    // in one v_dot2c, no byte extraction per state), where the block's LDS
    // then stays within 80 KB (two blocks per CU).  Channel mode only: B8 x
    // L2048 x 1536 channels, N32 0.380 -> 0.367 ms, N64 0.626 -> 0.614 ms;
    // the head layout (B4 x L8192, 24 heads x 64, N128) measured 2.466 ->
    // 2.512 ms with it (twice the LDS bytes per step for C)
    constexpr int kLdsC32 = CH * (kTC + 4) + 2 * kTC * N * 4 + (STAGE_Y ? kTC * CH * 4 : 16) + (DEFER ? kTC * CH * 8 : 8);
    constexpr bool C32 = WIDEB && MODE == kModeChannel && kLdsC32 <= 81920;
    __shared__ __align__(16) std::conditional_t<WIDEB, int32_t, int8_t> s_b[kTC][N];
    __shared__ __align__(16) std::conditional_t<C32, int32_t, int8_t> s_c[kTC][N];
    __shared__ __align__(16) int32_t s_o32[STAGE_Y ? kTC : 1][STAGE_Y ? CH : 4];
    __shared__ __align__(16) int2 s_y[DEFER ? kTC : 1][DEFER ? CH : 1];

    const int tid = threadIdx.x;
    const int ch = tid / G;
    const int g = tid % G;
    const int p0 = blockIdx.x * CH;
    const int hd = blockIdx.y;
    const int b = blockIdx.z;
    const int p = p0 + ch;
    const bool active = p < a.P;

    // ---- per-thread constants and state
    int32_t n2[S];  // 2n: the update16 form takes the doubled decay
    int32_t h[S];
    {
        const int64_t sidx = ((((int64_t)b * a.H + hd) * a.P + (active ? p : 0)) * N) + g * S;
        for (int s = 0; s < S; ++s) {
            h[s] = (a.h_in && active) ? a.h_in[sidx + s] : 0;
            if constexpr (MODE == kModeChannel)
                n2[s] = 2 * (active ? a.decay[(int64_t)p * N + g * S + s] : 0);
            else
                n2[s] = 2 * a.decay[hd];
        }
    }

    // ---- staging registers
    uint4 rx[XPER];
    uint4 rb[BCPER], rc[BCPER];
    const int64_t row0 = (int64_t)b * a.L;  // first (b, t=0) row index

    auto prefetch = [&](int t0) {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * kThreads;
            const int tt = i / X16, c16 = i % X16;
            const bool ok = i < XPIECES && t0 + tt < a.L && p0 + c16 * 16 < a.P;
            rx[j] = load16(a.x + (row0 + t0 + tt) * a.x_row + (int64_t)hd * a.P + p0 + c16 * 16, ok);
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * kThreads;
            const int tt = i / BC16, c16 = i % BC16;
            const bool ok = i < BCPIECES && t0 + tt < a.L;
            const int64_t off = (row0 + t0 + tt) * a.bc_row + (MODE == kModeHead ? (int64_t)hd * N : 0) + c16 * 16;
            rb[j] = load16(a.bsrc + off, ok);
            rc[j] = load16(a.csrc + off, ok);
        }
    };
    auto stash = [&]() {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * kThreads;
            if (i >= XPIECES) break;
            const int tt = i / X16, c16 = i % X16;
            const uint32_t w[4] = {rx[j].x, rx[j].y, rx[j].z, rx[j].w};
            for (int e = 0; e < 16; ++e) s_x[c16 * 16 + e][tt] = (int8_t)(w[e >> 2] >> (8 * (e & 3)));
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * kThreads;
            if (i >= BCPIECES) break;
            const int tt = i / BC16, c16 = i % BC16;
            if constexpr (WIDEB) {
                const uint32_t w[4] = {rb[j].x, rb[j].y, rb[j].z, rb[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<int4 *>(&s_b[tt][c16 * 16 + 4 * q]) =
                        make_int4(sbyte(w[q], 0), sbyte(w[q], 1), sbyte(w[q], 2), sbyte(w[q], 3));
            } else {
                *reinterpret_cast<uint4 *>(&s_b[tt][c16 * 16]) = rb[j];
            }
            if constexpr (C32) {
                const uint32_t w[4] = {rc[j].x, rc[j].y, rc[j].z, rc[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<int4 *>(&s_c[tt][c16 * 16 + 4 * q]) =
                        make_int4(sbyte(w[q], 0) * 65536, sbyte(w[q], 1) * 65536, sbyte(w[q], 2) * 65536,
                                  sbyte(w[q], 3) * 65536);
            } else {
                *reinterpret_cast<uint4 *>(&s_c[tt][c16 * 16]) = rc[j];
            }
        }
    };

    // one step of this lane's S states: the exact int32 partials of y
    auto step = [&](int t, int xv, int &yhi, int &ylo) {
        yhi = 0;
        ylo = 0;
        if constexpr (C32) {
            // every coefficient read first, then the S updates
            int bv[S], cv[S];
#pragma unroll
            for (int q = 0; q < S / 4; ++q) {
                const int4 b4 = *reinterpret_cast<const int4 *>(&s_b[t][g * S + 4 * q]);
                const int4 c4 = *reinterpret_cast<const int4 *>(&s_c[t][g * S + 4 * q]);
                bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
                cv[4 * q] = c4.x; cv[4 * q + 1] = c4.y; cv[4 * q + 2] = c4.z; cv[4 * q + 3] = c4.w;
            }
#pragma unroll
            for (int s = 0; s < S; ++s) update16_cs(h[s], n2[s], bv[s], xv, cv[s], yhi, ylo);
        } else if constexpr (WIDEB) {
            // every coefficient read first, then the S updates
            int bv[S];
            uint32_t cw[S / 4];
#pragma unroll
            for (int q = 0; q < S / 4; ++q) {
                const int4 b4 = *reinterpret_cast<const int4 *>(&s_b[t][g * S + 4 * q]);
                bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
                cw[q] = *reinterpret_cast<const uint32_t *>(&s_c[t][g * S + 4 * q]);
            }
#pragma unroll
            for (int s = 0; s < S; ++s) update16_b(h[s], n2[s], bv[s], xv, sbyte(cw[s >> 2], s & 3), yhi, ylo);
        } else {
            uint32_t bw = 0, cw = 0;
            for (int s = 0; s < S; ++s) {
                bw |= (uint32_t)(uint8_t)s_b[t][g * S + s] << (8 * s);
                cw |= (uint32_t)(uint8_t)s_c[t][g * S + s] << (8 * s);
            }
#pragma unroll
            for (int s = 0; s < S; ++s) update16(h[s], n2[s], __mul24(sbyte(bw, s), xv), sbyte(cw, s), yhi, ylo);
        }
    };

    const int nchunks = (a.L + kTC - 1) / kTC;
    prefetch(0);
    for (int cidx = 0; cidx < nchunks; ++cidx) {
        const int t0 = cidx * kTC;
        const int tn = min(kTC, a.L - t0);
        __syncthreads();
        stash();
        __syncthreads();
        if (cidx + 1 < nchunks) prefetch(t0 + kTC);

        for (int t4 = 0; t4 < tn; t4 += 4) {
            const uint32_t xw = *reinterpret_cast<const uint32_t *>(&s_x[ch][t4]);
            const int tend = min(4, tn - t4);
            if constexpr (DEFER) {
                if (tend == 4) {
                    // the eight partials of the group reduced stage by stage
                    // across all eight (no DPP wait states)
                    int y[8];
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt) step(t4 + tt, sbyte(xw, tt), y[2 * tt], y[2 * tt + 1]);
#pragma unroll
                    for (int q = 0; q < 8; ++q) if constexpr (G >= 2) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0xB1, 0xF, 0xF, false);
#pragma unroll
                    for (int q = 0; q < 8; ++q) if constexpr (G >= 4) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x4E, 0xF, 0xF, false);
#pragma unroll
                    for (int q = 0; q < 8; ++q) if constexpr (G >= 8) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x141, 0xF, 0xF, false);
#pragma unroll
                    for (int q = 0; q < 8; ++q) if constexpr (G >= 16) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x140, 0xF, 0xF, false);
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt) s_y[t4 + tt][ch] = make_int2(y[2 * tt], y[2 * tt + 1]);
                } else {
                    for (int tt = 0; tt < tend; ++tt) {
                        int yhi, ylo;
                        step(t4 + tt, sbyte(xw, tt), yhi, ylo);
                        s_y[t4 + tt][ch] = make_int2(group_sum<G>(yhi), group_sum<G>(ylo));
                    }
                }
                continue;
            }
            for (int tt = 0; tt < tend; ++tt) {
                const int t = t4 + tt;
                int yhi, ylo;
                step(t, sbyte(xw, tt), yhi, ylo);
                yhi = group_sum<G>(yhi);
                ylo = group_sum<G>(ylo);
                const int32_t y32 = sat32_64(((int64_t)yhi << 16) + ylo);
                if (g == 0) {
                    if constexpr (STAGE_Y) s_o32[t][ch] = y32;
                    else if (active) a.y[(row0 + t0 + t) * a.x_row + (int64_t)hd * a.P + p] = y32;
                }
            }
        }
        __syncthreads();
        if constexpr (DEFER) {
            // chunk epilogue: y = sat32(yhi * 2^16 + ylo)
            for (int i = tid; i < kTC * CH; i += kThreads) {
                const int tt = i / CH, cc = i % CH;
                if (tt < tn) {
                    const int2 yv = s_y[tt][cc];
                    s_o32[tt][cc] = sat32_64(((int64_t)yv.x << 16) + yv.y);
                }
            }
            __syncthreads();
        }
        // ---- write the staged outputs of this chunk
        if constexpr (STAGE_Y) {
            constexpr int Y4 = CH / 4;
            for (int i = tid; i < kTC * Y4; i += kThreads) {
                const int tt = i / Y4, c4 = i % Y4;
                if (tt < tn && p0 + c4 * 4 < a.P)
                    *reinterpret_cast<uint4 *>(a.y + (row0 + t0 + tt) * a.x_row + (int64_t)hd * a.P + p0 + c4 * 4) =
                        *reinterpret_cast<const uint4 *>(&s_o32[tt][c4 * 4]);
            }
        }
        if constexpr (MODE == kModeHead) {
            // chunk_states at every multiple of cs (cs is a multiple of kTC) and at the end
            const int tdone = t0 + tn;
            if (a.chunk_states && active && (tdone % a.cs == 0 || tdone == a.L)) {
                const int cc = (tdone - 1) / a.cs;
                int32_t *dst = a.chunk_states +
                               ((((int64_t)b * a.nchunks_out + cc) * a.H + hd) * a.P + p) * N + g * S;
                for (int s = 0; s < S; ++s) dst[s] = h[s];
            }
        }
    }
    if (a.h_out && active) {
        const int64_t sidx = ((((int64_t)b * a.H + hd) * a.P + p) * N) + g * S;
        for (int s = 0; s < S; ++s) a.h_out[sidx + s] = h[s];
    }
}

// ------------------------------------------ head mode, N = 128: mixed block
// At 16 lanes a channel (8 states a lane) a wave holds 4 channels; with B*H*P
// channels a multiple of 6 per SIMD (e.g. 4 x 24 heads x 64 = 6144 on 1024
// SIMDs) that leaves half the SIMDs two waves (8 channels) and the others one.
// Here a 512-thread block owns 24 consecutive channels of one sequence, flat
// over (head, p), so it may straddle two heads: waves 0-3 take 16 channels at
// 16 lanes a channel (8 states a lane), waves 4-7 take 8 channels at 32 lanes
// (4 states a lane).  Waves w and w + 4 of a block share a SIMD, so every SIMD
// runs 4 + 2 channels.  The two heads' B and C rows are staged side by side
// (B as int32 for the clamped multiply-add); the rest follows scan_kernel:
// 64-step chunks prefetched one chunk ahead, x transposed so one ds_read_b32
// serves 4 steps, four steps' y partials reduced together and recombined in a
// chunk epilogue, 16-byte output stores.
constexpr int kMixCH = 24, kMixCHA = 16;

template <int G>
__device__ __forceinline__ int group_sum_mix(int v) {
    v = group_sum<16>(v);
    if constexpr (G == 32) {
        // add the neighbouring 16-lane row: v_permlane16_swap exchanges rows 0/2
        // with rows 1/3, so the two results hold each lane's own and other row
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        v = (int)(r[0] + r[1]);
    }
    return v;
}

__global__ __launch_bounds__(512) void scan_head_mix_kernel(ScanArgs a) {
    constexpr int N = 128;
    constexpr int XP = kTC + 4;
    constexpr int NT = 512;
    __shared__ __align__(16) int8_t s_x[kMixCH][XP];
    __shared__ __align__(16) int32_t s_b[kTC][2 * N];
    __shared__ __align__(16) int8_t s_c[kTC][2 * N];
    __shared__ __align__(16) int32_t s_o32[kTC][kMixCH];
    __shared__ __align__(16) int2 s_y[kTC][kMixCH];

    const int tid = threadIdx.x;
    const bool wa = tid < 256;   // wave-uniform: a 16-lane (8-state) wave
    const int ch = wa ? tid / 16 : kMixCHA + (tid - 256) / 32;
    const int g = wa ? tid % 16 : (tid - 256) % 32;
    const int S = wa ? 8 : 4;
    const int c0 = blockIdx.x * kMixCH;   // first channel of the block, flat over (head, p)
    const int b = blockIdx.z;
    const int hd0 = c0 / a.P;
    const bool two = hd0 + 1 < a.H;        // a second head's B/C row exists
    const int cf = c0 + ch;
    const int hd = cf / a.P, p = cf - hd * a.P;
    const int boff = (hd - hd0) * N + g * S;   // this lane's first state in the staged B/C rows

    const int32_t n2 = 2 * a.decay[hd];
    int32_t h[8];
    const int64_t sidx = (((int64_t)b * a.H + hd) * a.P + p) * N + g * S;
#pragma unroll
    for (int s = 0; s < 8; ++s) h[s] = (a.h_in && s < S) ? a.h_in[sidx + s] : 0;

    // staging: x as 3 pieces of 8 bytes a step (192 a chunk), B and C as 16
    // pieces of 16 bytes a step over the two heads (1024 each, 2 a thread)
    uint2 rx;
    uint4 rb[2], rc[2];
    const int64_t row0 = (int64_t)b * a.L;
    auto prefetch = [&](int t0) {
        {
            const int tt = tid / 3, q = tid % 3;
            const bool ok = tid < kTC * 3 && t0 + tt < a.L;
            rx = ok ? *reinterpret_cast<const uint2 *>(a.x + (row0 + t0 + tt) * a.x_row + c0 + 8 * q) : make_uint2(0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = tid + j * NT;
            const int tt = i / 16, c16 = i % 16;
            const bool ok = t0 + tt < a.L && (c16 < 8 || two);
            const int64_t off = (row0 + t0 + tt) * a.bc_row + (int64_t)hd0 * N + c16 * 16;
            rb[j] = load16(a.bsrc + off, ok);
            rc[j] = load16(a.csrc + off, ok);
        }
    };
    auto stash = [&]() {
        if (tid < kTC * 3) {
            const int tt = tid / 3, q = tid % 3;
            const uint32_t w[2] = {rx.x, rx.y};
#pragma unroll
            for (int e = 0; e < 8; ++e) s_x[8 * q + e][tt] = (int8_t)(w[e >> 2] >> (8 * (e & 3)));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = tid + j * NT;
            const int tt = i / 16, c16 = i % 16;
            const uint32_t w[4] = {rb[j].x, rb[j].y, rb[j].z, rb[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<int4 *>(&s_b[tt][c16 * 16 + 4 * q]) =
                    make_int4(sbyte(w[q], 0), sbyte(w[q], 1), sbyte(w[q], 2), sbyte(w[q], 3));
            *reinterpret_cast<uint4 *>(&s_c[tt][c16 * 16]) = rc[j];
        }
    };
    // one step of this lane's SS states: the exact int32 partials of y
    auto step = [&](auto ss, int t, int xv, int &yhi, int &ylo) {
        constexpr int SS = decltype(ss)::value;
        yhi = 0;
        ylo = 0;
        int bv[SS];
        uint32_t cw[SS / 4];
#pragma unroll
        for (int q = 0; q < SS / 4; ++q) {
            const int4 b4 = *reinterpret_cast<const int4 *>(&s_b[t][boff + 4 * q]);
            bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
            cw[q] = *reinterpret_cast<const uint32_t *>(&s_c[t][boff + 4 * q]);
        }
#pragma unroll
        for (int s = 0; s < SS; ++s) update16_b(h[s], n2, bv[s], xv, sbyte(cw[s >> 2], s & 3), yhi, ylo);
    };
    // four steps (or the chunk's last tend < 4) of one wave kind
    auto group = [&](auto ss, int t4, int tend, uint32_t xw) {
        constexpr int SS = decltype(ss)::value, GG = 128 / SS;
        if (tend == 4) {
            int y[8];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) step(ss, t4 + tt, sbyte(xw, tt), y[2 * tt], y[2 * tt + 1]);
#pragma unroll
            for (int q = 0; q < 8; ++q) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0xB1, 0xF, 0xF, false);
#pragma unroll
            for (int q = 0; q < 8; ++q) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x4E, 0xF, 0xF, false);
#pragma unroll
            for (int q = 0; q < 8; ++q) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x141, 0xF, 0xF, false);
#pragma unroll
            for (int q = 0; q < 8; ++q) y[q] += __builtin_amdgcn_update_dpp(0, y[q], 0x140, 0xF, 0xF, false);
            if constexpr (GG == 32) {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)y[q], (unsigned)y[q], false, false);
                    y[q] = (int)(r[0] + r[1]);
                }
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) s_y[t4 + tt][ch] = make_int2(y[2 * tt], y[2 * tt + 1]);
        } else {
            for (int tt = 0; tt < tend; ++tt) {
                int yhi, ylo;
                step(ss, t4 + tt, sbyte(xw, tt), yhi, ylo);
                s_y[t4 + tt][ch] = make_int2(group_sum_mix<GG>(yhi), group_sum_mix<GG>(ylo));
            }
        }
    };

    const int nchunks = (a.L + kTC - 1) / kTC;
    prefetch(0);
    for (int cidx = 0; cidx < nchunks; ++cidx) {
        const int t0 = cidx * kTC;
        const int tn = min(kTC, a.L - t0);
        __syncthreads();
        stash();
        __syncthreads();
        if (cidx + 1 < nchunks) prefetch(t0 + kTC);
        for (int t4 = 0; t4 < tn; t4 += 4) {
            const uint32_t xw = *reinterpret_cast<const uint32_t *>(&s_x[ch][t4]);
            const int tend = min(4, tn - t4);
            if (wa)
                group(std::integral_constant<int, 8>{}, t4, tend, xw);
            else
                group(std::integral_constant<int, 4>{}, t4, tend, xw);
        }
        __syncthreads();
        // chunk epilogue: y = sat32(yhi * 2^16 + ylo), then 16-byte stores of the 24 channels' rows
        for (int i = tid; i < kTC * kMixCH; i += NT) {
            const int tt = i / kMixCH, cc = i % kMixCH;
            if (tt < tn) {
                const int2 yv = s_y[tt][cc];
                s_o32[tt][cc] = sat32_64(((int64_t)yv.x << 16) + yv.y);
            }
        }
        __syncthreads();
        for (int i = tid; i < kTC * (kMixCH / 4); i += NT) {
            const int tt = i / (kMixCH / 4), c4 = i % (kMixCH / 4);
            if (tt < tn)
                *reinterpret_cast<uint4 *>(a.y + (row0 + t0 + tt) * a.x_row + c0 + c4 * 4) =
                    *reinterpret_cast<const uint4 *>(&s_o32[tt][c4 * 4]);
        }
        // chunk_states at every multiple of cs (cs is a multiple of kTC) and at the end
        const int tdone = t0 + tn;
        if (a.chunk_states && (tdone % a.cs == 0 || tdone == a.L)) {
            const int cc = (tdone - 1) / a.cs;
            int32_t *dst = a.chunk_states + ((((int64_t)b * a.nchunks_out + cc) * a.H + hd) * a.P + p) * N + g * S;
#pragma unroll
            for (int s = 0; s < 8; ++s)
                if (s < S) dst[s] = h[s];
        }
    }
    if (a.h_out) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
            if (s < S) a.h_out[sidx + s] = h[s];
    }
}

// ---------------------------------------------------------------- generic
// Plain int64 kernels for every shape the fast kernel does not take, and for
// chunk lengths that are not multiples of the staging chunk.  One thread per
// (b, head, channel), all states in a loop, inputs read straight from global.
template <int MODE>
__global__ __launch_bounds__(256) void scan_generic_kernel(ScanArgs a, int N) {
    const int64_t lane = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lanes = (int64_t)a.B * a.H * a.P;
    if (lane >= lanes) return;
    const int p = (int)(lane % a.P);
    const int hd = (int)((lane / a.P) % a.H);
    const int b = (int)(lane / ((int64_t)a.P * a.H));
    int32_t h[128];
    const int64_t sidx = (((int64_t)b * a.H + hd) * a.P + p) * N;
    for (int n = 0; n < N; ++n) h[n] = a.h_in ? a.h_in[sidx + n] : 0;
    for (int t = 0; t < a.L; ++t) {
        const int64_t rr = (int64_t)b * a.L + t;
        int64_t xv;
        int dmv = 0;
        const int8_t *brow, *crow;
        if constexpr (MODE == kModeModel) {
            dmv = clamp32(a.dm[rr * a.x_row + p], -20, 20);
            xv = rshr64((int64_t)a.x[rr * a.x_row + p] * dt_q16(dmv), 10);
            brow = a.bsrc + rr * a.bc_row;
            crow = a.csrc + rr * a.bc_row;
        } else {
            xv = a.x[rr * a.x_row + (int64_t)hd * a.P + p];
            brow = a.bsrc + rr * a.bc_row + (MODE == kModeHead ? (int64_t)hd * N : 0);
            crow = a.csrc + rr * a.bc_row + (MODE == kModeHead ? (int64_t)hd * N : 0);
        }
        int64_t acc = 0;
        for (int n = 0; n < N; ++n) {
            int64_t nd;
            if constexpr (MODE == kModeChannel) nd = a.decay[(int64_t)p * N + n];
            else if constexpr (MODE == kModeHead) nd = a.decay[hd];
            else nd = clamp64((int64_t)a.decay[(int64_t)p * N + n] + dmv, 0, 32000);
            const int64_t dec = ((int64_t)h[n] * nd) >> a.k;
            h[n] = sat32_64(dec + (int64_t)brow[n] * xv);
            acc += (int64_t)crow[n] * h[n];
        }
        const int32_t y32 = sat32_64(acc);
        if constexpr (MODE == kModeModel) {
            const int zv = a.z[rr * a.z_row + p];
            const int64_t yg = ((int64_t)y32 * gate_q15(zv)) >> 15;
            a.yo[rr * a.x_row + p] = (int8_t)clamp64(rshr64(yg, a.s_y), -127, 127);
        } else {
            a.y[rr * a.x_row + (int64_t)hd * a.P + p] = y32;
        }
        if constexpr (MODE == kModeHead) {
            if (a.chunk_states && ((t + 1) % a.cs == 0 || t + 1 == a.L)) {
                const int cc = t / a.cs;
                int32_t *dst = a.chunk_states + ((((int64_t)b * a.nchunks_out + cc) * a.H + hd) * a.P + p) * N;
                for (int n = 0; n < N; ++n) dst[n] = h[n];
            }
        }
    }
    if (a.h_out)
        for (int n = 0; n < N; ++n) a.h_out[sidx + n] = h[n];
}

// ------------------------------------------------------------- dispatch
// Lanes per channel: enough waves to cover the 1024 SIMDs when possible.
int pick_g(int N, int64_t channels) {
    int g = 1;
    while (g < 16 && N % (2 * g) == 0 && (N / g > 32 || channels * g / 64 < 1024)) g *= 2;
    return g;
}

template <int N, int MODE>
hipError_t launch_fast_n(int G, const ScanArgs &a, hipStream_t st) {
    auto grid = [&](int ch) { return dim3((unsigned)((a.P + ch - 1) / ch), (unsigned)a.H, (unsigned)a.B); };
    switch (G) {
#define MI_CASE_G(GG)                                                                   \
    case GG:                                                                            \
        if constexpr (N / GG >= 1 && N / GG <= 32) {                                    \
            hipLaunchKernelGGL((scan_kernel<N, GG, MODE>), grid(kThreads / GG), dim3(kThreads), 0, st, a); \
            return hipGetLastError();                                                   \
        }                                                                               \
        break;
        MI_CASE_G(1)
        MI_CASE_G(2)
        MI_CASE_G(4)
        MI_CASE_G(8)
        MI_CASE_G(16)
#undef MI_CASE_G
    }
    return hipErrorInvalidValue;
}

template <int MODE>
hipError_t launch_scan(const ScanArgs &a, int N, bool fast, hipStream_t st) {
    // (the model mode's fast shapes run model_scan_kernel; here it takes the
    // generic kernel only)
    if constexpr (MODE != kModeModel) {
        if (fast) {
            const int G = pick_g(N, (int64_t)a.B * a.H * a.P);
            switch (N) {
                case 16: return launch_fast_n<16, MODE>(G, a, st);
                case 32: return launch_fast_n<32, MODE>(G, a, st);
                case 64: return launch_fast_n<64, MODE>(G, a, st);
                case 128: return launch_fast_n<128, MODE>(G, a, st);
            }
        }
    }
    const int64_t lanes = (int64_t)a.B * a.H * a.P;
    hipLaunchKernelGGL((scan_generic_kernel<MODE>), dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st, a, N);
    return hipGetLastError();
}

bool fast_shape(int N, int P, int k, int mode) {
    if (N != 16 && N != 32 && N != 64 && !(N == 128 && mode != kModeModel)) return false;
    if (P % 16 != 0) return false;
    // k = 15 only: n2 = 2n <= 2^16 keeps L*n2 below 2^32 and H*n2 in int32.
    return k == 15;
}

// ------------------------------------------------ float-compat reference
// Exact semantics of the reference launch_dyadic_scan
// (dyadic_mamba_kernel.cu:35-63): one lane per (b, d), int64 state.
__global__ __launch_bounds__(256) void scan_f32_kernel(const float *x, const int32_t *nums, const int32_t *shifts,
                                                       float *h, int B, int S, int D, int sb) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)B * D) return;
    const int d = (int)(idx % D);
    const int b = (int)(idx / D);
    const float scale_f = (float)((long long)1 << sb);
    long long hc = 0;
    for (int t = 0; t < S; ++t) {
        const int64_t off = ((int64_t)b * S + t) * D + d;
        const float xs = x[off] * scale_f;
        const long long xf = (long long)xs;
        hc = hc * (long long)nums[off];
        hc = hc >> shifts[off];
        hc += xf;
        h[off] = (float)hc / scale_f;
    }
}

// Elementwise integer recurrence: one lane per (b, channel), int32 state.
__global__ __launch_bounds__(256) void scan_elem_kernel(const int32_t *u, const int32_t *n, int k, int32_t *h,
                                                        const int32_t *h_in, int32_t *h_out, int B, int L, int C) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)B * C) return;
    const int c = (int)(idx % C);
    const int b = (int)(idx / C);
    int32_t s = h_in ? h_in[idx] : 0;
    for (int t = 0; t < L; ++t) {
        const int64_t off = ((int64_t)b * L + t) * C + c;
        s = sat32_64((((int64_t)s * n[off]) >> k) + (int64_t)u[off]);
        h[off] = s;
    }
    if (h_out) h_out[idx] = s;
}

// Chunked elementwise recurrence with the per-chunk outputs of
// ssd_chunked_scan_forward (ssd_chunked_scan.py:382-422): one lane per
// (b, channel), its steps in order.  The operands of kAhead steps are loaded
// before the dependent chain runs over them, from clamped in-bounds addresses
// (no per-lane condition, so the loads issue back to back); a step past the
// end is skipped by a branch that is uniform across the block.  At the end of
// each chunk the lane stores its state and the chunk's cumulative decay in
// Q30 (2^30 decayed by the chunk's steps, rounded down after each step).
constexpr int kAhead = 8;
__global__ __launch_bounds__(64) void chunked_scan_kernel(const int32_t *__restrict__ u, const int32_t *__restrict__ n,
                                                          int k, int cs, int32_t *__restrict__ h,
                                                          int32_t *__restrict__ final_h, int32_t *__restrict__ dte,
                                                          const int32_t *h_in, int32_t *h_out, int B, int L, int C,
                                                          int nc) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)B * C) return;
    const int c = (int)(idx % C);
    const int b = (int)(idx / C);
    const int64_t base = (int64_t)b * L * C + c;
    int32_t s = h_in ? h_in[idx] : 0;
    int32_t p = 1 << 30;
    int left = cs;     // steps left in the current chunk
    int chunk = 0;
    for (int t0 = 0; t0 < L; t0 += kAhead) {
        int32_t uu[kAhead], nn[kAhead];
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
            const int64_t off = base + (int64_t)min(t0 + j, L - 1) * C;
            uu[j] = u[off];
            nn[j] = n[off];
        }
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
            const int t = t0 + j;
            if (t < L) {
                s = sat32_64((((int64_t)s * nn[j]) >> k) + (int64_t)uu[j]);
                h[base + (int64_t)t * C] = s;
                p = sat32_64(((int64_t)p * nn[j]) >> k);
                if (--left == 0 || t + 1 == L) {
                    const int64_t co = ((int64_t)b * nc + chunk) * C + c;
                    if (final_h) final_h[co] = s;
                    if (dte) dte[co] = p;
                    p = 1 << 30;
                    left = cs;
                    ++chunk;
                }
            }
        }
    }
    if (h_out) h_out[idx] = s;
}

}  // namespace

hipError_t launch_model_scan(const int8_t *xs, const int8_t *dm, const int8_t *z, const int8_t *bsrc,
                             const int8_t *csrc, const int32_t *base, int8_t *yo, const int32_t *h_in, int32_t *h_out,
                             int64_t x_row, int64_t z_row, int64_t bc_row, int B, int L, int D, int N, int s_y,
                             hipStream_t st);
hipError_t launch_ssd_scan(const int8_t *xs, const int8_t *xp, const int8_t *z, const int32_t *tab, int8_t *yo,
                           const int32_t *h_in, int32_t *h_out, int64_t x_row, int64_t xp_row, int64_t z_row, int B,
                           int L, int H, int P, int N, int s_y, hipStream_t st);
}  // namespace mi

using namespace mi;

extern "C" mi_status mi_dyadic_scan(const int8_t *x, const int8_t *b, const int8_t *c, const int32_t *decay_num,
                                    int decay_shift, int32_t *y, const int32_t *h_in, int32_t *h_out, int batch,
                                    int len, int d, int nstate, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && d >= 0, MI_ERR_BAD_DIM, "mi_dyadic_scan: negative size");
    MI_REQUIRE(nstate >= 1 && nstate <= 128, MI_ERR_BAD_DIM, "mi_dyadic_scan: nstate=%d outside [1,128]", nstate);
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 16, MI_ERR_BAD_ARG, "mi_dyadic_scan: decay_shift=%d outside [1,16]",
               decay_shift);
    if ((int64_t)batch * d == 0) return MI_OK;
    MI_REQUIRE(decay_num && y, MI_ERR_NULL_POINTER, "mi_dyadic_scan: decay_num and y are required");
    if (len > 0) MI_REQUIRE(x && b && c, MI_ERR_NULL_POINTER, "mi_dyadic_scan: x, b and c are required");
    ScanArgs a{};
    a.x = x; a.bsrc = b; a.csrc = c; a.decay = decay_num; a.y = y; a.h_in = h_in; a.h_out = h_out;
    a.x_row = d; a.bc_row = nstate; a.B = batch; a.L = len; a.H = 1; a.P = d; a.k = decay_shift;
    const bool fast = len > 0 && fast_shape(nstate, d, decay_shift, kModeChannel) && aligned(x, 16) && aligned(b, 16) &&
                      aligned(c, 16) && aligned(y, 16);
    if (len == 0 && !h_out) return MI_OK;
    hipError_t e = launch_scan<kModeChannel>(a, nstate, fast, as_stream(stream));
    if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_dyadic_scan: launch failed: %s", hipGetErrorString(e));
    return MI_OK;
}

extern "C" mi_status mi_ssd_chunked_scan(const int8_t *x, const int8_t *b, const int8_t *c, const int32_t *decay_num,
                                         int decay_shift, int32_t *y, int32_t *chunk_states, const int32_t *h_in,
                                         int32_t *h_out, int batch, int len, int heads, int head_dim, int nstate,
                                         int chunk, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && heads >= 0 && head_dim >= 0, MI_ERR_BAD_DIM,
               "mi_ssd_chunked_scan: negative size");
    MI_REQUIRE(nstate >= 1 && nstate <= 128, MI_ERR_BAD_DIM, "mi_ssd_chunked_scan: nstate=%d outside [1,128]", nstate);
    MI_REQUIRE(chunk >= 1, MI_ERR_BAD_ARG, "mi_ssd_chunked_scan: chunk=%d must be >= 1", chunk);
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 16, MI_ERR_BAD_ARG,
               "mi_ssd_chunked_scan: decay_shift=%d outside [1,16]", decay_shift);
    if ((int64_t)batch * heads * head_dim == 0 || (len == 0 && !h_out)) return MI_OK;
    MI_REQUIRE(decay_num && (len == 0 || (x && b && c && y)), MI_ERR_NULL_POINTER,
               "mi_ssd_chunked_scan: x, b, c, decay_num, y required");
    ScanArgs a{};
    a.x = x; a.bsrc = b; a.csrc = c; a.decay = decay_num; a.y = y; a.chunk_states = chunk_states;
    a.h_in = h_in; a.h_out = h_out;
    a.x_row = (int64_t)heads * head_dim; a.bc_row = (int64_t)heads * nstate;
    a.B = batch; a.L = len; a.H = heads; a.P = head_dim; a.k = decay_shift;
    a.cs = chunk; a.nchunks_out = (len + chunk - 1) / chunk;
    const bool fast = len > 0 && fast_shape(nstate, head_dim, decay_shift, kModeHead) && (chunk % kTC == 0) && aligned(x, 16) &&
                      aligned(b, 16) && aligned(c, 16) && aligned(y, 16);
    // the mixed 24-channel block where its blocks fill every CU exactly (one
    // block per CU at a time: 102 KB of LDS)
    const int64_t hp = (int64_t)heads * head_dim, mix_blocks = hp / kMixCH * batch;
    const bool mix = fast && nstate == 128 && hp % kMixCH == 0 && head_dim >= kMixCH && hp / kMixCH <= 65535 &&
                     mix_blocks % device_cus() == 0;
    hipError_t e;
    if (mix) {
        hipLaunchKernelGGL(scan_head_mix_kernel, dim3((unsigned)(hp / kMixCH), 1u, (unsigned)batch), dim3(512), 0,
                           as_stream(stream), a);
        e = hipGetLastError();
    } else {
        e = launch_scan<kModeHead>(a, nstate, fast, as_stream(stream));
    }
    if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_ssd_chunked_scan: launch failed: %s", hipGetErrorString(e));
    return MI_OK;
}

extern "C" mi_status mi_block_scan(const int8_t *xs, const int8_t *dm, const int8_t *xp, int xp_stride, int b_off,
                                   const int8_t *z, int z_stride, int z_off, const int32_t *base, int decay_shift,
                                   int s_y, int8_t *yo, const int32_t *h_in, int32_t *h_out, int batch, int len,
                                   int d_inner, int nstate, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_block_scan: negative size");
    MI_REQUIRE(nstate >= 1 && nstate <= 64, MI_ERR_BAD_DIM, "mi_block_scan: nstate=%d outside [1,64]", nstate);
    MI_REQUIRE(decay_shift == 15, MI_ERR_BAD_ARG, "mi_block_scan: decay_shift=%d, the model path uses 15", decay_shift);
    MI_REQUIRE(s_y >= 0 && s_y <= 30, MI_ERR_BAD_ARG, "mi_block_scan: s_y=%d outside [0,30]", s_y);
    MI_REQUIRE(b_off >= 0 && b_off + 2 * nstate <= xp_stride, MI_ERR_BAD_DIM,
               "mi_block_scan: B/C columns [%d,%d) exceed xp_stride=%d", b_off, b_off + 2 * nstate, xp_stride);
    MI_REQUIRE(z_off >= 0 && z_off + d_inner <= z_stride, MI_ERR_BAD_DIM,
               "mi_block_scan: z columns exceed z_stride=%d", z_stride);
    if ((int64_t)batch * d_inner == 0 || (len == 0 && !h_out)) return MI_OK;
    MI_REQUIRE(base && (len == 0 || (xs && dm && xp && z && yo)), MI_ERR_NULL_POINTER,
               "mi_block_scan: a required pointer is NULL");
    ScanArgs a{};
    a.x = xs; a.dm = dm; a.z = z + z_off; a.bsrc = xp + b_off; a.csrc = xp + b_off + nstate; a.decay = base;
    a.yo = yo; a.h_in = h_in; a.h_out = h_out;
    a.x_row = d_inner; a.bc_row = xp_stride; a.z_row = z_stride;
    a.B = batch; a.L = len; a.H = 1; a.P = d_inner; a.k = decay_shift; a.s_y = s_y;
    const bool fast = len > 0 && fast_shape(nstate, d_inner, decay_shift, kModeModel) && aligned(xs, 16) && aligned(dm, 16) &&
                      aligned(a.z, 16) && aligned(a.bsrc, 16) && aligned(a.csrc, 16) && aligned(yo, 16) &&
                      xp_stride % 16 == 0 && z_stride % 16 == 0;
    hipError_t e;
    if (fast && nstate != 128)
        e = launch_model_scan(xs, dm, a.z, a.bsrc, a.csrc, base, yo, h_in, h_out, d_inner, z_stride, xp_stride, batch,
                              len, d_inner, nstate, s_y, as_stream(stream));
    else
        e = launch_scan<kModeModel>(a, nstate, fast, as_stream(stream));
    if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_block_scan: launch failed: %s", hipGetErrorString(e));
    return MI_OK;
}

extern "C" mi_status mi_ssd_block_scan(const int8_t *xs, const int8_t *xp, int xp_stride, const int8_t *z,
                                       int z_stride, int z_off, const int32_t *decay_tab, int n_heads, int s_y,
                                       int8_t *yo, const int32_t *h_in, int32_t *h_out, int batch, int len,
                                       int d_inner, int nstate, void *stream) {
    const char *fn = "mi_ssd_block_scan";
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && d_inner >= 0 && n_heads >= 1, MI_ERR_BAD_DIM, "%s: bad size", fn);
    MI_REQUIRE(nstate == 16 || nstate == 32 || nstate == 64, MI_ERR_BAD_DIM, "%s: nstate=%d (16, 32 or 64)", fn,
               nstate);
    MI_REQUIRE(d_inner % n_heads == 0 && (d_inner / n_heads) % 16 == 0, MI_ERR_BAD_DIM,
               "%s: d_inner=%d must split into %d heads of a multiple of 16 channels", fn, d_inner, n_heads);
    MI_REQUIRE(s_y >= 0 && s_y <= 30, MI_ERR_BAD_ARG, "%s: s_y=%d outside [0,30]", fn, s_y);
    MI_REQUIRE(xp_stride >= 2 * n_heads * nstate + n_heads && xp_stride % 16 == 0, MI_ERR_BAD_DIM,
               "%s: xp_stride=%d must hold B, C and dt of every head and be a multiple of 16", fn, xp_stride);
    MI_REQUIRE(z_off >= 0 && z_off + d_inner <= z_stride && z_stride % 16 == 0 && z_off % 16 == 0, MI_ERR_BAD_DIM,
               "%s: z columns [%d,%d) and stride %d (multiples of 16)", fn, z_off, z_off + d_inner, z_stride);
    if ((int64_t)batch * d_inner == 0 || (len == 0 && !h_out)) return MI_OK;
    MI_REQUIRE(decay_tab && (len == 0 || (xs && xp && z && yo)), MI_ERR_NULL_POINTER, "%s: a required pointer is NULL",
               fn);
    MI_REQUIRE(len == 0 || (aligned(xs, 16) && aligned(xp, 16) && aligned(z, 16) && aligned(yo, 16)),
               MI_ERR_BAD_ALIGNMENT, "%s: xs, xp, z and yo must be 16-byte aligned", fn);
    MI_REQUIRE(aligned(h_in, 4) && aligned(h_out, 4) && aligned(decay_tab, 4), MI_ERR_BAD_ALIGNMENT,
               "%s: h_in, h_out and decay_tab must be 4-byte aligned", fn);
    const hipError_t e = launch_ssd_scan(xs, xp, z + z_off, decay_tab, yo, h_in, h_out, d_inner, xp_stride, z_stride,
                                         batch, len, n_heads, d_inner / n_heads, nstate, s_y, as_stream(stream));
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return MI_OK;
}

extern "C" mi_status mi_dyadic_scan_f32(const float *x, const int32_t *nums, const int32_t *shifts, float *h,
                                        int batch, int seq, int dim, int scale_bits, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && seq >= 0 && dim >= 0, MI_ERR_BAD_DIM, "mi_dyadic_scan_f32: negative size");
    MI_REQUIRE(scale_bits >= 0 && scale_bits <= 62, MI_ERR_BAD_ARG, "mi_dyadic_scan_f32: scale_bits=%d outside [0,62]",
               scale_bits);
    if ((int64_t)batch * seq * dim == 0) return MI_OK;
    MI_REQUIRE(x && nums && shifts && h, MI_ERR_NULL_POINTER, "mi_dyadic_scan_f32: a required pointer is NULL");
    const int64_t lanes = (int64_t)batch * dim;
    hipLaunchKernelGGL(scan_f32_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, as_stream(stream), x,
                       nums, shifts, h, batch, seq, dim, scale_bits);
    return check_launch("mi_dyadic_scan_f32");
}

extern "C" mi_status mi_dyadic_scan_elementwise(const int32_t *u, const int32_t *nums, int decay_shift, int32_t *h,
                                                const int32_t *h_in, int32_t *h_out, int batch, int len, int channels,
                                                void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && channels >= 0, MI_ERR_BAD_DIM, "mi_dyadic_scan_elementwise: negative size");
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 30, MI_ERR_BAD_ARG,
               "mi_dyadic_scan_elementwise: decay_shift=%d outside [1,30]", decay_shift);
    // len == 0 with h_out: the kernel runs no step and writes h_out = h_in (zeros when NULL)
    if ((int64_t)batch * channels == 0 || (len == 0 && !h_out)) return MI_OK;
    MI_REQUIRE(len == 0 || (u && nums && h), MI_ERR_NULL_POINTER,
               "mi_dyadic_scan_elementwise: u, nums and h are required");
    const int64_t lanes = (int64_t)batch * channels;
    hipLaunchKernelGGL(scan_elem_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, as_stream(stream), u,
                       nums, decay_shift, h, h_in, h_out, batch, len, channels);
    return check_launch("mi_dyadic_scan_elementwise");
}

extern "C" mi_status mi_dyadic_chunked_scan(const int32_t *u, const int32_t *nums, int decay_shift, int chunk,
                                            int32_t *h, int32_t *final_h, int32_t *decay_to_end, const int32_t *h_in,
                                            int32_t *h_out, int batch, int len, int channels, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && channels >= 0, MI_ERR_BAD_DIM, "mi_dyadic_chunked_scan: negative size");
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 30, MI_ERR_BAD_ARG,
               "mi_dyadic_chunked_scan: decay_shift=%d outside [1,30]", decay_shift);
    MI_REQUIRE(chunk >= 1, MI_ERR_BAD_ARG, "mi_dyadic_chunked_scan: chunk=%d must be >= 1", chunk);
    // len == 0 with h_out: the kernel runs no step and writes h_out = h_in (zeros when NULL)
    if ((int64_t)batch * channels == 0 || (len == 0 && !h_out)) return MI_OK;
    MI_REQUIRE(len == 0 || (u && nums && h), MI_ERR_NULL_POINTER, "mi_dyadic_chunked_scan: u, nums and h are required");
    const int64_t lanes = (int64_t)batch * channels;
    const int nc = (int)((len + (int64_t)chunk - 1) / chunk);
    hipLaunchKernelGGL(chunked_scan_kernel, dim3((unsigned)((lanes + 63) / 64)), dim3(64), 0, as_stream(stream), u,
                       nums, decay_shift, chunk, h, final_h, decay_to_end, h_in, h_out, batch, len, channels, nc);
    return check_launch("mi_dyadic_chunked_scan");
}
