// Fused model scan for prefill on gfx950 (spec mi-spec-2, rules 4.7-4.11):
// decay from base + dm, dt from dm, input xs*dt (x) B, the exact floor
// recurrence, y = C.h, the gate by z and the requant of the out_proj input.
//
// Layout: a block of NT threads owns CH = NT/G channels of one sequence; G
// adjacent lanes share a channel and keep S = N/G states each in VGPRs (read
// as two 16-bit fields by the update, update16).  The mixed block puts half
// its threads in layout G and half in a layout G2 > G (at N = 16: 32 channels
// of 8 lanes, then 16 of 16 lanes): where batch x d_inner gives 1 to 1.5
// waves of 8-lane channels per SIMD, one such block per CU loads every SIMD
// with the same work instead of leaving half of them with twice the rest.
// Per chunk of 64 steps the block stages xs, dm, z (transposed to
// channel-major bytes) and B, C (widened to int32 so a state
// reads its coefficients with one ds_read_b128 per four states) through LDS,
// in two buffers where they fit: chunk c+1 is staged right after chunk c's
// steps, and its global loads were issued a whole chunk earlier.
//
// The per-step work of a lane is only the recurrence and two exact int32
// partial sums of y.  Steps run in groups of four: the next group's B and C
// are read from LDS into the other of two register sets while this group's
// recurrence runs, and the group's eight partial sums are combined over the
// channel's G lanes stage by stage across all eight (DPP adds whose sources
// were written several instructions earlier, so no wait states).  The
// epilogue (recombine, saturate, gate, requant) runs once per (step, channel)
// at the end of the chunk, spread over all threads.
// Per update: decay 1 (2*base + 2*dm), decay term 3 (two SDWA multiplies, an
// SDWA add), input and saturating add 1 (a clamped v_mad_i32_i24), y partials
// 2 (a v_dot2c and a multiply) and their adds, decay clamp 0-1 (skipped when
// every base of the wave lies at least 20 inside [0, 32000], where base + dm
// cannot leave the range).
#include <type_traits>

#include "mi_common.hpp"
#include "mi_mfma.hpp"

namespace mi {
namespace {

constexpr int kMThreads = 256;
constexpr int kMTC = 64;  // steps per staged chunk

template <int G>
__device__ __forceinline__ int msum(int v) {
    // every source lane is valid for these patterns, so bound_ctrl lets each
    // stage be a single v_add_u32_dpp
    if constexpr (G >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);   // quad_perm 1,0,3,2
    if constexpr (G >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);   // quad_perm 2,3,0,1
    if constexpr (G >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    if constexpr (G >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true); // row_mirror
    return v;
}

__device__ __forceinline__ int sb(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }

struct MScanArgs {
    const int8_t *xs, *dm, *z;     // [B*L rows][row stride]
    const int8_t *bsrc, *csrc;     // B, C rows (row stride bc_row)
    const int32_t *base;           // [D][N]
    int8_t *yo;                    // [B*L][D]
    const int32_t *h_in;
    int32_t *h_out;
    int64_t x_row, z_row, bc_row;
    int B, L, D, s_y;
};

// DPP sums of K independent values over the G lanes of a channel, stage by
// stage across all K values: a DPP add then reads a register written K
// instructions earlier, so no wait states are needed between the stages.
template <int G, int K>
__device__ __forceinline__ void msum_all(int (&v)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k)
        if constexpr (G >= 2) v[k] += __builtin_amdgcn_update_dpp(0, v[k], 0xB1, 0xF, 0xF, true);
#pragma unroll
    for (int k = 0; k < K; ++k)
        if constexpr (G >= 4) v[k] += __builtin_amdgcn_update_dpp(0, v[k], 0x4E, 0xF, 0xF, true);
#pragma unroll
    for (int k = 0; k < K; ++k)
        if constexpr (G >= 8) v[k] += __builtin_amdgcn_update_dpp(0, v[k], 0x141, 0xF, 0xF, true);
#pragma unroll
    for (int k = 0; k < K; ++k)
        if constexpr (G >= 16) v[k] += __builtin_amdgcn_update_dpp(0, v[k], 0x140, 0xF, 0xF, true);
}

// G2 = 0: every lane of the block in layout G.  G2 > G: threads [0, NT/2)
// in layout G and [NT/2, NT) in layout G2 (fewer states a lane), the block's
// first CHA channels in the first; with one block per CU and waves dealt to
// the four SIMDs in turn, every SIMD then holds one wave of each.
template <int N, int G, int NT, int G2 = 0>
__global__ __launch_bounds__(NT) void model_scan_kernel(MScanArgs a) {
    constexpr bool MIX = G2 > 0;
    constexpr int NTA = MIX ? NT / 2 : NT;           // threads of layout G
    constexpr int CHA = NTA / G;
    constexpr int CH = CHA + (MIX ? (NT - NTA) / G2 : 0);
    constexpr int S = N / G;                          // the most states a lane holds
    static_assert(!MIX || (G2 > G && NTA % 64 == 0 && N % G2 == 0), "mixed layout");
    constexpr int XP = kMTC + 4;
    constexpr int X16 = CH / 16;
    constexpr int XPIECES = kMTC * X16;
    constexpr int XPER = (XPIECES + NT - 1) / NT;
    constexpr int BC16 = N / 16;
    constexpr int BCPIECES = kMTC * BC16;
    constexpr int BCPER = (BCPIECES + NT - 1) / NT;
    static_assert(N % 16 == 0 && CH % 16 == 0 && (S == 1 || S == 2 || S % 4 == 0), "state split");
    static_assert(!MIX || N / G2 == 1 || N / G2 == 2 || (N / G2) % 4 == 0, "state split");
    // The mixed block (its CU to itself, 160 KB of LDS) reduces each step's y
    // partials only within quads of lanes and leaves the channel's quad sums
    // in LDS, PW slots a channel (slots a layout of G/4 < PW quads never
    // writes stay zero), for the chunk epilogue to add: two DPP stages a step
    // fewer for 16 lanes, one for 8.  It stages xd as int32 (no unpacking per
    // step).  The other layouts reduce over all G lanes and stage xd as int16.
    constexpr int PA = MIX && G >= 8 ? G / 4 : 1;     // quads of a channel, layout G
    constexpr int PB = MIX && G2 >= 8 ? G2 / 4 : 1;   // and layout G2
    constexpr int PW = PA > PB ? PA : PB;             // y partial slots per channel
    constexpr int YW = CH * PW;                       // y partials per step
    using XdT = std::conditional_t<MIX, int32_t, int16_t>;
    // staging buffers: two (chunk c + 1 is staged while chunk c's epilogue runs)
    // where they fit in 64 KB of LDS (160 KB for a mixed block), else one
    constexpr int kStage = 2 * CH * XP + CH * XP * (int)sizeof(XdT) + 2 * (kMTC + 4) * N * 4;
    constexpr int kLds = MIX ? 163840 : 65536;   // a mixed block has its CU to itself
    constexpr int kFixed = kMTC * (YW * 8 + CH) + 297 * 4;
    constexpr int NB = 2 * kStage + kFixed <= kLds ? 2 : 1;
    static_assert(NB * kStage + kFixed <= kLds, "LDS budget");

    // One LDS block with the arrays every step reads first, so their addresses
    // stay below 64 KB, within a ds instruction's immediate offset (placed
    // after the 98 KB of y partials, each look-ahead read needed an add).
    // B and C have four rows past the chunk: the last group's look-ahead
    // reads them and discards what it read, so the reads need no clamped row.
    struct Smem {
        int32_t b[NB][kMTC + 4][N];
        int32_t c[NB][kMTC + 4][N];
        int8_t x[NB][2][CH][XP];    // 2*dm, z (channel-major)
        XdT xd[NB][CH][XP];         // rshr(xs * dt(dm), 10), |xd| <= 813
        int2 y[kMTC][YW];           // (yhi, ylo) partials per step
        int8_t o[kMTC][CH];
        int32_t dt[41];
        int32_t gate[256];
    };
    __shared__ __align__(16) Smem sm;
    auto &s_b = sm.b;
    auto &s_c = sm.c;
    auto &s_x = sm.x;
    auto &s_xd = sm.xd;
    auto &s_y = sm.y;
    auto &s_o = sm.o;
    auto &s_dt = sm.dt;
    auto &s_gate = sm.gate;

    const int tid = threadIdx.x;
    const bool second = MIX && tid >= NTA;                     // wave-uniform
    constexpr int GB = MIX ? G2 : G;
    const int SL = second ? N / GB : S;                        // this lane's states
    const int ch = second ? CHA + (tid - NTA) / GB : tid / G;
    const int g = second ? (tid - NTA) % GB : tid % G;
    const int p0 = blockIdx.x * CH;
    const int b = blockIdx.y;
    const int p = p0 + ch;
    const bool active = p < a.D;
    // this lane's y partial: its channel's slots, its quad (g / 4 < PW)
    const int yslot = ch * PW + (PW > 1 ? g / 4 : 0);
    // the chunk epilogue's channel and first step for this thread
    constexpr int TPC = NT / CH;
    const int ecc = tid % CH, et1 = tid / CH;

    for (int i = tid; i < 41; i += NT) s_dt[i] = dt_q16(i - 20);
    for (int i = tid; i < 256; i += NT) s_gate[i] = gate_q15(i - 128);

    int32_t base2[S], h[S];  // 2 * base: the update takes n2 = 2n
    bool safe = true;
    {
        const int64_t sidx = ((int64_t)b * a.D + (active ? p : 0)) * N + g * SL;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const bool own = s < SL;
            h[s] = (a.h_in && active && own) ? a.h_in[sidx + s] : 0;
            const int32_t bs = active && own ? a.base[(int64_t)p * N + g * SL + s] : 16000;
            base2[s] = 2 * bs;
            safe = safe && bs >= 20 && bs <= 32000 - 20;
        }
    }
    // a wave-uniform choice: every lane of the wave can drop the decay clamp
    const bool wave_safe = __all(safe);

    // ext_vector_type registers (a union-typed uint4 array touched through
    // lambdas is kept in scratch)
    v4i rx[3][XPER];
    v4i rb[BCPER], rc[BCPER];
    const int64_t row0 = (int64_t)b * a.L;
    auto prefetch = [&](int t0) {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * NT;
            const int tt = i / X16, c16 = i % X16;
            const bool ok = i < XPIECES && t0 + tt < a.L && p0 + c16 * 16 < a.D;
            const int64_t rr = row0 + t0 + tt;
            const v4i zero = v4i{0, 0, 0, 0};
            rx[0][j] = ok ? *reinterpret_cast<const v4i *>(a.xs + rr * a.x_row + p0 + c16 * 16) : zero;
            rx[1][j] = ok ? *reinterpret_cast<const v4i *>(a.dm + rr * a.x_row + p0 + c16 * 16) : zero;
            rx[2][j] = ok ? *reinterpret_cast<const v4i *>(a.z + rr * a.z_row + p0 + c16 * 16) : zero;
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * NT;
            const int tt = i / BC16, c16 = i % BC16;
            const bool ok = i < BCPIECES && t0 + tt < a.L;
            const int64_t off = (row0 + t0 + tt) * a.bc_row + c16 * 16;
            rb[j] = ok ? *reinterpret_cast<const v4i *>(a.bsrc + off) : v4i{0, 0, 0, 0};
            rc[j] = ok ? *reinterpret_cast<const v4i *>(a.csrc + off) : v4i{0, 0, 0, 0};
        }
    };
    auto stash = [&](int bf) {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * NT;
            if (i >= XPIECES) break;
            const int tt = i / X16, c16 = i % X16;
            const uint32_t wx[4] = {(uint32_t)rx[0][j][0], (uint32_t)rx[0][j][1], (uint32_t)rx[0][j][2],
                                    (uint32_t)rx[0][j][3]};
            const uint32_t wd[4] = {(uint32_t)rx[1][j][0], (uint32_t)rx[1][j][1], (uint32_t)rx[1][j][2],
                                    (uint32_t)rx[1][j][3]};
            const uint32_t wz[4] = {(uint32_t)rx[2][j][0], (uint32_t)rx[2][j][1], (uint32_t)rx[2][j][2],
                                    (uint32_t)rx[2][j][3]};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int dmv = clamp32(sb(wd[e >> 2], e & 3), -20, 20);
                s_x[bf][0][c16 * 16 + e][tt] = (int8_t)(2 * dmv);  // the decay takes 2n
                s_x[bf][1][c16 * 16 + e][tt] = (int8_t)sb(wz[e >> 2], e & 3);
                // |x| <= 128, dt <= 6554: a 24-bit product
                s_xd[bf][c16 * 16 + e][tt] = (XdT)((__mul24(sb(wx[e >> 2], e & 3), s_dt[dmv + 20]) + 512) >> 10);
            }
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * NT;
            if (i >= BCPIECES) break;
            const int tt = i / BC16, c16 = i % BC16;
            const uint32_t wb[4] = {(uint32_t)rb[j][0], (uint32_t)rb[j][1], (uint32_t)rb[j][2], (uint32_t)rb[j][3]};
            const uint32_t wc[4] = {(uint32_t)rc[j][0], (uint32_t)rc[j][1], (uint32_t)rc[j][2], (uint32_t)rc[j][3]};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s_b[bf][tt][c16 * 16 + e] = sb(wb[e >> 2], e & 3);
                s_c[bf][tt][c16 * 16 + e] = sb(wc[e >> 2], e & 3) * 65536;  // C * 2^16 (update16_cs)
            }
        }
    };

    // this lane's SS coefficients of B and C for step t (LDS row t < kMTC)
    auto load_bc = [&](int bf, int t, auto &bv, auto &cv) {
        constexpr int SS = sizeof(bv) / sizeof(int);
        if constexpr (SS >= 4) {
#pragma unroll
            for (int q = 0; q < SS / 4; ++q) {
                const int4 b4 = *reinterpret_cast<const int4 *>(&s_b[bf][t][g * SS + 4 * q]);
                const int4 c4 = *reinterpret_cast<const int4 *>(&s_c[bf][t][g * SS + 4 * q]);
                bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
                cv[4 * q] = c4.x; cv[4 * q + 1] = c4.y; cv[4 * q + 2] = c4.z; cv[4 * q + 3] = c4.w;
            }
        } else if constexpr (SS == 2) {
            const int2 b2 = *reinterpret_cast<const int2 *>(&s_b[bf][t][g * SS]);
            const int2 c2 = *reinterpret_cast<const int2 *>(&s_c[bf][t][g * SS]);
            bv[0] = b2.x; bv[1] = b2.y; cv[0] = c2.x; cv[1] = c2.y;
        } else {
            bv[0] = s_b[bf][t][g];
            cv[0] = s_c[bf][t][g];
        }
    };
    // the recurrence of this lane's SS states for one step: returns the exact
    // int32 partials (sum C*H, sum C*L) of y over the lane's states (the first
    // state's products start the sums: no zeroed accumulator)
    auto update = [&](int xd, int dm2, const auto &bv, const auto &cs, int &yhi, int &ylo, auto clamp_tag) {
        constexpr bool CLAMP = decltype(clamp_tag)::value;
        constexpr int SS = sizeof(bv) / sizeof(int);
#pragma unroll
        for (int s = 0; s < SS; ++s) {
            const int n2 = CLAMP ? clamp32(base2[s] + dm2, 0, 64000) : base2[s] + dm2;
            if (s == 0) update16_cs_first(h[s], n2, bv[s], xd, cs[s], yhi, ylo);
            else update16_cs(h[s], n2, bv[s], xd, cs[s], yhi, ylo);
        }
    };

    // Per chunk: the steps of chunk c, (two buffers) the staging of chunk c+1,
    // a barrier, the epilogue of chunk c (recombine, saturate, gate, requant)
    // into s_o, a barrier, the 16-byte stores of chunk c and the global loads
    // of the chunk after next.  One buffer: chunk c+1 is staged after the
    // stores, behind a third barrier.
    const int nchunks = (a.L + kMTC - 1) / kMTC;
    if constexpr (PA < PW) {
        // the layout-G channels' slots [PA, PW), never written by their lanes
        constexpr int kz = CHA * (PW - PA);
        for (int i = tid; i < kMTC * kz; i += NT) {
            const int tt = i / kz, r = i - tt * kz;
            s_y[tt][(r / (PW - PA)) * PW + PA + r % (PW - PA)] = make_int2(0, 0);
        }
    }
    prefetch(0);
    stash(0);
    if (nchunks > 1) prefetch(kMTC);
    __syncthreads();
    for (int cidx = 0; cidx < nchunks; ++cidx) {
        const int t0 = cidx * kMTC;  // chunk start
        const int tn = min(kMTC, a.L - t0);
        const int cur = NB == 2 ? (cidx & 1) : 0;

        auto run_chunk = [&](auto clamp_tag, auto g_tag) {
            constexpr int GG = decltype(g_tag)::value, SS = N / GG;
            constexpr int GQ = MIX && GG >= 8 ? 4 : GG;   // lanes a step's y is reduced over
            const int t4n = tn & ~3;  // steps in whole groups of four
            // groups of four steps: the next group's coefficients, 2*dm and xd
            // are read from LDS while this group's recurrence runs, and the y
            // partials of the four steps are reduced together afterwards; two
            // register sets alternate between the groups of a pair (reads past
            // the chunk land in the staging arrays' four padding steps)
            auto load_dx = [&](int t4, uint32_t &dw, int (&xdv)[4]) {
                dw = *reinterpret_cast<const uint32_t *>(&s_x[cur][0][ch][t4]);
                if constexpr (MIX) {
                    const int4 xw = *reinterpret_cast<const int4 *>(&s_xd[cur][ch][t4]);
                    xdv[0] = xw.x; xdv[1] = xw.y; xdv[2] = xw.z; xdv[3] = xw.w;
                } else {
                    const uint2 xw = *reinterpret_cast<const uint2 *>(&s_xd[cur][ch][t4]);
                    xdv[0] = (int)(int16_t)xw.x; xdv[1] = (int)xw.x >> 16;
                    xdv[2] = (int)(int16_t)xw.y; xdv[3] = (int)xw.y >> 16;
                }
            };
            auto group = [&](int t4, const int (&bq)[4][SS], const int (&cq)[4][SS], const uint32_t dq,
                             const int (&xq)[4], int (&bn)[4][SS], int (&cn)[4][SS], uint32_t &dn, int (&xn)[4]) {
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) load_bc(cur, t4 + 4 + tt, bn[tt], cn[tt]);
                load_dx(t4 + 4, dn, xn);
                int y[8];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt)
                    update(xq[tt], sb(dq, tt), bq[tt], cq[tt], y[2 * tt], y[2 * tt + 1], clamp_tag);
                msum_all<GQ>(y);
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) s_y[t4 + tt][yslot] = make_int2(y[2 * tt], y[2 * tt + 1]);
            };
            int b0[4][SS], c0[4][SS], b1[4][SS], c1[4][SS], x0[4], x1[4];
            uint32_t d0, d1;
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) load_bc(cur, tt, b0[tt], c0[tt]);
            load_dx(0, d0, x0);
            for (int t4 = 0; t4 < t4n; t4 += 8) {
                group(t4, b0, c0, d0, x0, b1, c1, d1, x1);
                if (t4 + 4 < t4n) group(t4 + 4, b1, c1, d1, x1, b0, c0, d0, x0);
            }
            for (int t = t4n; t < tn; ++t) {
                int bv[SS], cv[SS];
                load_bc(cur, t, bv, cv);
                const int dm2 = s_x[cur][0][ch][t];
                int y[2];
                update(s_xd[cur][ch][t], dm2, bv, cv, y[0], y[1], clamp_tag);
                msum_all<GQ>(y);
                s_y[t][yslot] = make_int2(y[0], y[1]);  // the lanes of a quad hold the same sums: no branch
            }
        };
        using GA = std::integral_constant<int, G>;
        using GBT = std::integral_constant<int, GB>;
        if (second) {
            if constexpr (MIX) {
                if (wave_safe) run_chunk(std::false_type{}, GBT{});
                else run_chunk(std::true_type{}, GBT{});
            }
        } else {
            if (wave_safe) run_chunk(std::false_type{}, GA{});
            else run_chunk(std::true_type{}, GA{});
        }
        if constexpr (NB == 2)
            if (cidx + 1 < nchunks) stash(cur ^ 1);
        __syncthreads();
        // epilogue of the chunk: y = sat32(yhi*2^16 + ylo), gate, requant; a
        // thread keeps one channel and walks the chunk's steps t1, t1 + TPC, ...
        if (tid < TPC * CH) {
#pragma unroll
            for (int k = 0; k < (kMTC + TPC - 1) / TPC; ++k) {
                const int tw = et1 + k * TPC;
                const int tt = min(tw, kMTC - 1);   // reads stay in the chunk; the store below checks tw
                int yh = 0, yl = 0;
#pragma unroll
                for (int q = 0; q < PW; ++q) {
                    const int2 w = s_y[tt][ecc * PW + q];
                    yh += w.x;
                    yl += w.y;
                }
                // y = hi * 2^16 + (yl mod 2^16) exactly (|yh|, |yl| < 2^28), and
                // y fits int32 exactly when hi does in 16 bits
                const int hi = yh + (yl >> 16);
                const int hc = clamp32(hi, -32768, 32767);
                int32_t y32 = (int32_t)(((uint32_t)hc << 16) | ((uint32_t)yl & 0xffffu));
                if (hi != hc) y32 = hi > 0 ? INT32_MAX : INT32_MIN;
                const int zv = s_x[cur][1][ecc][tt];
                const int32_t gt = s_gate[zv + 128];   // in [0, 2^15]
                // floor(y32 * gt / 2^15) with 24-bit products: y32 = yh15 * 2^15 +
                // yl15, |yh15| <= 2^16, 0 <= yl15 < 2^15 (|result| <= |y32|)
                const int32_t yh15 = y32 >> 15, yl15 = y32 & 0x7fff;
                const int32_t yg = __mul24(yh15, gt) + (int32_t)(__umul24((uint32_t)yl15, (uint32_t)gt) >> 15);
                // rshr(yg, s_y) exactly in 32 bits: floor(yg / 2^s) plus bit s-1
                const int32_t qv = a.s_y > 0 ? (yg >> a.s_y) + ((yg >> (a.s_y - 1)) & 1) : yg;
                if (tw < tn) s_o[tw][ecc] = (int8_t)clamp32(qv, -127, 127);
            }
        }
        __syncthreads();
        for (int i = tid; i < kMTC * X16; i += NT) {
            const int tt = i / X16, c16 = i % X16;
            if (tt < tn && p0 + c16 * 16 < a.D)
                *reinterpret_cast<uint4 *>(a.yo + (row0 + t0 + tt) * a.x_row + p0 + c16 * 16) =
                    *reinterpret_cast<const uint4 *>(&s_o[tt][c16 * 16]);
        }
        if constexpr (NB == 2) {
            if (cidx + 2 < nchunks) prefetch(t0 + 2 * kMTC);
        } else if (cidx + 1 < nchunks) {
            stash(0);
            if (cidx + 2 < nchunks) prefetch(t0 + 2 * kMTC);
            __syncthreads();
        }
    }
    if (a.h_out && active) {
        const int64_t sidx = ((int64_t)b * a.D + p) * N + g * SL;
#pragma unroll
        for (int s = 0; s < S; ++s)
            if (s < SL) a.h_out[sidx + s] = h[s];
    }
}

template <int N, int G, int NT>
hipError_t launch_model_ngt(const MScanArgs &a, hipStream_t st) {
    constexpr int CH = NT / G;
    if constexpr (4 * CH * (kMTC + 4) + 2 * kMTC * N * 4 + kMTC * CH * 9 + 297 * 4 <= 65536) {
        // (one staging buffer fits; the kernel doubles it where two fit)
        hipLaunchKernelGGL((model_scan_kernel<N, G, NT>), dim3((unsigned)((a.D + CH - 1) / CH), (unsigned)a.B),
                           dim3(NT), 0, st, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

// The mixed block: NT/2 threads in layout G, NT/2 in layout G2.
template <int N, int G, int G2, int NT>
hipError_t launch_model_mix(const MScanArgs &a, hipStream_t st) {
    constexpr int CH = NT / 2 / G + NT / 2 / G2;
    hipLaunchKernelGGL((model_scan_kernel<N, G, NT, G2>), dim3((unsigned)((a.D + CH - 1) / CH), (unsigned)a.B),
                       dim3(NT), 0, st, a);
    return hipGetLastError();
}

template <int N>
hipError_t launch_model_n(int G, int NT, const MScanArgs &a, hipStream_t st) {
#define MI_MCASE(GG, TT) \
    if (G == GG && NT == TT) return launch_model_ngt<N, GG, TT>(a, st);
    MI_MCASE(4, 256)
    MI_MCASE(8, 256)
    MI_MCASE(16, 256)
#undef MI_MCASE
    return hipErrorInvalidValue;
}

// ------------------------------------------------ SSD block scan (V2)
// The scan of MambaIntegerBlockV2 (spec rules 7.4-7.8; ssd_multihead.py:
// 536-586): per (sequence, head) a P x N state with one decay per step and
// head, h = floor(h * n_t / 2^15) + Bq[n] * x[p], y = sum_n Cq[n] h, clamp,
// gate, requant.  Same lane layout as model_scan_kernel (G lanes per channel,
// S = N/G states each, the update16 step); a block's CH channels lie in
// one head.  Per chunk the block stages x and z (channel-major), the step
// decays (table lookup of the head's dt column) and B, C: each 16-byte piece
// of a token's B (or C) row sums its squares, the token's N/16 pieces (lanes
// of one quad) add up by DPP, and every piece is scaled to the unit vector in
// Q7 before it lands in LDS, so the steps read finished coefficients.
struct SScanArgs {
    const int8_t *xs, *z, *xp;     // [B*L rows][row stride]; z points at its first column
    const int32_t *tab;            // [H][255]
    int8_t *yo;
    const int32_t *h_in;
    int32_t *h_out;
    int64_t x_row, z_row, xp_row;
    int B, L, D, H, P, s_y;
};

// Q7 unit-vector scale of spec rule 7.4 from the row's sum of squares
__device__ __forceinline__ int32_t unit_inv(int32_t ss) {
    if (ss == 0) return 0;
    const uint32_t nrm = (uint32_t)isqrt64((uint64_t)ss << 16);
    return (int32_t)((1u << 30) / nrm);
}

template <int N, int G>
__global__ __launch_bounds__(kMThreads) void ssd_scan_kernel(SScanArgs a) {
    constexpr int S = N / G;
    constexpr int CH = kMThreads / G;
    constexpr int XP = kMTC + 4;
    constexpr int X16 = CH / 16;
    constexpr int XPIECES = kMTC * X16;
    constexpr int XPER = (XPIECES + kMThreads - 1) / kMThreads;
    constexpr int BC16 = N / 16;
    constexpr int BCPIECES = kMTC * BC16;
    constexpr int BCPER = (BCPIECES + kMThreads - 1) / kMThreads;
    static_assert(N % 16 == 0 && BC16 <= 4 && (S == 1 || S == 2 || S % 4 == 0), "state split");
    static_assert(BCPIECES % 64 == 0 || BCPIECES < 64, "whole waves stage B and C");

    __shared__ __align__(16) int8_t s_x[2][CH][XP];        // xs, z (channel-major)
    __shared__ __align__(16) int32_t s_b[kMTC][N];
    __shared__ __align__(16) int32_t s_c[kMTC][N];          // C * 2^16 (update16_cs)
    __shared__ __align__(16) int2 s_y[kMTC][CH];
    __shared__ __align__(16) int8_t s_o[kMTC][CH];
    __shared__ __align__(16) int32_t s_n[kMTC];
    __shared__ int32_t s_tab[256];
    __shared__ int32_t s_gate[256];

    const int tid = threadIdx.x;
    const int ch = tid / G;
    const int g = tid % G;
    const int p0 = blockIdx.x * CH;
    const int head = p0 / a.P;
    const int b = blockIdx.y;
    const int p = p0 + ch;

    // doubled: the update takes n2 = 2n (table entries lie in [0, 2^15])
    for (int i = tid; i < 255; i += kMThreads) s_tab[i] = 2 * a.tab[(int64_t)head * 255 + i];
    for (int i = tid; i < 256; i += kMThreads) s_gate[i] = gate_q15(i - 128);

    int32_t h[S];
    {
        const int64_t sidx = ((int64_t)b * a.D + p) * N + g * S;
        for (int s = 0; s < S; ++s) h[s] = a.h_in ? a.h_in[sidx + s] : 0;
    }

    // ext_vector_type registers (a union-typed uint4 array touched through
    // lambdas is kept in scratch)
    v4i rx[2][XPER];
    v4i rb[BCPER], rc[BCPER];
    int dtv = 0;
    const int64_t row0 = (int64_t)b * a.L;
    const int64_t b_col = (int64_t)head * N, c_col = (int64_t)a.H * N + head * N, dt_col = 2 * (int64_t)a.H * N + head;
    auto prefetch = [&](int t0) {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * kMThreads;
            const int tt = i / X16, c16 = i % X16;
            const bool ok = i < XPIECES && t0 + tt < a.L;
            const int64_t rr = row0 + t0 + tt;
            const v4i zero = v4i{0, 0, 0, 0};
            rx[0][j] = ok ? *reinterpret_cast<const v4i *>(a.xs + rr * a.x_row + p0 + c16 * 16) : zero;
            rx[1][j] = ok ? *reinterpret_cast<const v4i *>(a.z + rr * a.z_row + p0 + c16 * 16) : zero;
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * kMThreads;
            const int tt = i / BC16, c16 = i % BC16;
            const bool ok = i < BCPIECES && t0 + tt < a.L;
            const int64_t off = (row0 + t0 + tt) * a.xp_row + c16 * 16;
            rb[j] = ok ? *reinterpret_cast<const v4i *>(a.xp + off + b_col) : v4i{0, 0, 0, 0};
            rc[j] = ok ? *reinterpret_cast<const v4i *>(a.xp + off + c_col) : v4i{0, 0, 0, 0};
        }
        dtv = (tid < kMTC && t0 + tid < a.L) ? a.xp[(row0 + t0 + tid) * a.xp_row + dt_col] : 0;
    };
    // sum of squares of a 16-byte piece of int8
    auto sumsq = [](v4i v) {
        const uint32_t w[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
        int ss = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int q = sb(w[e >> 2], e & 3);
            ss += q * q;
        }
        return ss;
    };
    auto stash = [&]() {
        for (int j = 0; j < XPER; ++j) {
            const int i = tid + j * kMThreads;
            if (i >= XPIECES) break;
            const int tt = i / X16, c16 = i % X16;
            const uint32_t wx[4] = {(uint32_t)rx[0][j][0], (uint32_t)rx[0][j][1], (uint32_t)rx[0][j][2],
                                    (uint32_t)rx[0][j][3]};
            const uint32_t wz[4] = {(uint32_t)rx[1][j][0], (uint32_t)rx[1][j][1], (uint32_t)rx[1][j][2],
                                    (uint32_t)rx[1][j][3]};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s_x[0][c16 * 16 + e][tt] = (int8_t)sb(wx[e >> 2], e & 3);
                s_x[1][c16 * 16 + e][tt] = (int8_t)sb(wz[e >> 2], e & 3);
            }
        }
        for (int j = 0; j < BCPER; ++j) {
            const int i = tid + j * kMThreads;
            if (i - (tid & 63) >= BCPIECES) break;  // whole waves: the DPP sums below need every lane
            const int tt = i / BC16, c16 = i % BC16;
            // the token's pieces are BC16 adjacent lanes of one quad
            int sbq = sumsq(rb[j]), scq = sumsq(rc[j]);
            if constexpr (BC16 >= 2) {
                sbq += __builtin_amdgcn_update_dpp(0, sbq, 0xB1, 0xF, 0xF, true);
                scq += __builtin_amdgcn_update_dpp(0, scq, 0xB1, 0xF, 0xF, true);
            }
            if constexpr (BC16 >= 4) {
                sbq += __builtin_amdgcn_update_dpp(0, sbq, 0x4E, 0xF, 0xF, true);
                scq += __builtin_amdgcn_update_dpp(0, scq, 0x4E, 0xF, 0xF, true);
            }
            const int32_t ib = unit_inv(sbq), ic = unit_inv(scq);
            const uint32_t wb[4] = {(uint32_t)rb[j][0], (uint32_t)rb[j][1], (uint32_t)rb[j][2], (uint32_t)rb[j][3]};
            const uint32_t wc[4] = {(uint32_t)rc[j][0], (uint32_t)rc[j][1], (uint32_t)rc[j][2], (uint32_t)rc[j][3]};
            if (i < BCPIECES) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    s_b[tt][c16 * 16 + e] = clamp32(rshr32(sb(wb[e >> 2], e & 3) * ib, 15), -127, 127);
                    s_c[tt][c16 * 16 + e] = clamp32(rshr32(sb(wc[e >> 2], e & 3) * ic, 15), -127, 127) * 65536;
                }
            }
        }
        if (tid < kMTC) s_n[tid] = s_tab[clamp32(dtv, -127, 127) + 127];
    };

    // one step of this lane's S states: the exact int32 partials of y (the
    // channel's G lanes are summed per group of four steps below)
    auto step = [&](int t, int xv, int n2, int &yhi, int &ylo) {
        int bv[S], cv[S];
        if constexpr (S >= 4) {
            for (int q = 0; q < S / 4; ++q) {
                const int4 b4 = *reinterpret_cast<const int4 *>(&s_b[t][g * S + 4 * q]);
                const int4 c4 = *reinterpret_cast<const int4 *>(&s_c[t][g * S + 4 * q]);
                bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
                cv[4 * q] = c4.x; cv[4 * q + 1] = c4.y; cv[4 * q + 2] = c4.z; cv[4 * q + 3] = c4.w;
            }
        } else {
            for (int s = 0; s < S; ++s) {
                bv[s] = s_b[t][g * S + s];
                cv[s] = s_c[t][g * S + s];
            }
        }
        yhi = 0;
        ylo = 0;
        for (int s = 0; s < S; ++s) update16_cs(h[s], n2, bv[s], xv, cv[s], yhi, ylo);
    };

    const int32_t ylim = 100 << 18;
    const int nchunks = (a.L + kMTC - 1) / kMTC;
    prefetch(0);
    for (int cidx = 0; cidx < nchunks; ++cidx) {
        const int t0 = cidx * kMTC;
        const int tn = min(kMTC, a.L - t0);
        __syncthreads();
        stash();
        __syncthreads();
        if (cidx + 1 < nchunks) prefetch(t0 + kMTC);
        for (int t4 = 0; t4 < tn; t4 += 4) {
            const uint32_t xw = *reinterpret_cast<const uint32_t *>(&s_x[0][ch][t4]);
            const int4 n4 = *reinterpret_cast<const int4 *>(&s_n[t4]);
            const int nv[4] = {n4.x, n4.y, n4.z, n4.w};
            if (t4 + 4 <= tn) {
                // the eight partials of the group reduced stage by stage across
                // all eight: each DPP add reads a register written several
                // instructions earlier, so it needs no wait states
                int y[8];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) step(t4 + tt, sb(xw, tt), nv[tt], y[2 * tt], y[2 * tt + 1]);
                msum_all<G>(y);
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) s_y[t4 + tt][ch] = make_int2(y[2 * tt], y[2 * tt + 1]);
            } else {
                for (int tt = 0; tt < tn - t4; ++tt) {
                    int y[2];
                    step(t4 + tt, sb(xw, tt), s_n[t4 + tt], y[0], y[1]);
                    msum_all<G>(y);
                    s_y[t4 + tt][ch] = make_int2(y[0], y[1]);
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < kMTC * CH; i += kMThreads) {
            const int tt = i / CH, cc = i % CH;
            if (tt < tn) {
                const int2 yv = s_y[tt][cc];
                const int32_t y32 = clamp32(sat32_64(((int64_t)yv.x << 16) + yv.y), -ylim, ylim);
                const int32_t gt = s_gate[s_x[1][cc][tt] + 128];
                const int32_t yh = y32 >> 15, yl = y32 & 0x7fff;
                const int32_t yg = yh * gt + (int32_t)(((uint32_t)yl * (uint32_t)gt) >> 15);
                s_o[tt][cc] = (int8_t)clamp64(rshr64(yg, a.s_y), -127, 127);
            }
        }
        __syncthreads();
        for (int i = tid; i < kMTC * X16; i += kMThreads) {
            const int tt = i / X16, c16 = i % X16;
            if (tt < tn)
                *reinterpret_cast<uint4 *>(a.yo + (row0 + t0 + tt) * a.x_row + p0 + c16 * 16) =
                    *reinterpret_cast<const uint4 *>(&s_o[tt][c16 * 16]);
        }
    }
    if (a.h_out) {
        const int64_t sidx = ((int64_t)b * a.D + p) * N + g * S;
        for (int s = 0; s < S; ++s) a.h_out[sidx + s] = h[s];
    }
}

// One step of the SSD block scan (decode, len 1): block = 256/G channels of one
// (sequence, head), G lanes per channel with S = N/G states each (the head's
// P x N state is 16 KB at P = N = 64).  Wave 0 builds the token's unit-vector B and C (Q7)
// and the step decay in LDS while every lane loads its states; then the same
// split update, y partials, DPP sum, clamp, gate and requant as ssd_scan_kernel.
template <int N, int S>
__global__ __launch_bounds__(kMThreads) void ssd_step_kernel(SScanArgs a) {
    constexpr int G = N / S;
    static_assert(G == 4 || G == 8 || G == 16, "lanes per channel");
    __shared__ int32_t s_b[N], s_c[N];
    __shared__ int32_t s_nt;
    const int tid = threadIdx.x;
    const int ch = tid / G, g = tid % G;
    const int b = blockIdx.y;
    const int p0 = blockIdx.x * (kMThreads / G);  // P % (256 / G) == 0 (checked by the launcher)
    const int head = p0 / a.P;
    const int p = p0 + ch;
    const int64_t row = (int64_t)b * a.L;  // L == 1
    const int64_t sidx = ((int64_t)b * a.D + p) * N + g * S;
    int32_t hv[S];
    if constexpr (S % 4 == 0) {
#pragma unroll
        for (int q = 0; q < S / 4; ++q) {
            const int4 h4 = a.h_in ? *reinterpret_cast<const int4 *>(a.h_in + sidx + 4 * q) : make_int4(0, 0, 0, 0);
            hv[4 * q] = h4.x; hv[4 * q + 1] = h4.y; hv[4 * q + 2] = h4.z; hv[4 * q + 3] = h4.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < S; ++q) hv[q] = a.h_in ? a.h_in[sidx + q] : 0;
    }
    const int xv = a.xs[row * a.x_row + p];
    const int zv = a.z[row * a.z_row + p];
    if (tid < 64) {
        // lane n < N: B[n], C[n] of the head; the squares summed over the wave
        const int8_t *xp = a.xp + row * a.xp_row;
        const int n = min(tid, N - 1);
        const int bn = tid < N ? xp[(int64_t)head * N + n] : 0;
        const int cn = tid < N ? xp[(int64_t)a.H * N + head * N + n] : 0;
        int sb2 = bn * bn, sc2 = cn * cn;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            sb2 += __shfl_xor(sb2, off);
            sc2 += __shfl_xor(sc2, off);
        }
        const int32_t ib = unit_inv(sb2), ic = unit_inv(sc2);
        if (tid < N) {
            s_b[tid] = clamp32(rshr32(bn * ib, 15), -127, 127);
            s_c[tid] = clamp32(rshr32(cn * ic, 15), -127, 127);
        }
        if (tid == 0) {
            const int dtv = xp[2 * (int64_t)a.H * N + head];
            s_nt = a.tab[(int64_t)head * 255 + clamp32(dtv, -127, 127) + 127];
        }
    }
    __syncthreads();
    const int n2 = 2 * s_nt;  // table entries lie in [0, 2^15]
    int yhi = 0, ylo = 0;
    int32_t hn[S];
#pragma unroll
    for (int q = 0; q < S; ++q) {
        hn[q] = hv[q];
        update16_b(hn[q], n2, s_b[g * S + q], xv, s_c[g * S + q], yhi, ylo);
    }
    if (a.h_out) {
        if constexpr (S % 4 == 0) {
#pragma unroll
            for (int q = 0; q < S / 4; ++q)
                *reinterpret_cast<int4 *>(a.h_out + sidx + 4 * q) =
                    make_int4(hn[4 * q], hn[4 * q + 1], hn[4 * q + 2], hn[4 * q + 3]);
        } else {
#pragma unroll
            for (int q = 0; q < S; ++q) a.h_out[sidx + q] = hn[q];
        }
    }
    yhi = msum<G>(yhi);
    ylo = msum<G>(ylo);
    if (g == 0) {
        const int32_t ylim = 100 << 18;
        const int32_t y32 = clamp32(sat32_64(((int64_t)yhi << 16) + ylo), -ylim, ylim);
        const int32_t gt = gate_q15(zv);
        const int32_t yh = y32 >> 15, yl = y32 & 0x7fff;
        const int32_t yg = yh * gt + (int32_t)(((uint32_t)yl * (uint32_t)gt) >> 15);
        a.yo[row * a.x_row + p] = (int8_t)clamp64(rshr64(yg, a.s_y), -127, 127);
    }
}

}  // namespace

// Used by mi_ssd_block_scan: N in {16, 32, 64}, d_head % 16 == 0, 16-byte
// aligned rows.  Lanes per channel: the split that keeps S = 4 states per
// lane where it can (16 at N = 64, 8 at N = 32, 4 at N = 16), narrowed so a
// block's channels stay in one head.
hipError_t launch_ssd_scan(const int8_t *xs, const int8_t *xp, const int8_t *z, const int32_t *tab, int8_t *yo,
                           const int32_t *h_in, int32_t *h_out, int64_t x_row, int64_t xp_row, int64_t z_row, int B,
                           int L, int H, int P, int N, int s_y, hipStream_t st) {
    SScanArgs a{};
    a.xs = xs; a.xp = xp; a.z = z; a.tab = tab; a.yo = yo; a.h_in = h_in; a.h_out = h_out;
    a.x_row = x_row; a.xp_row = xp_row; a.z_row = z_row;
    a.B = B; a.L = L; a.D = H * P; a.H = H; a.P = P; a.s_y = s_y;
    if (L == 1 && aligned(h_in, 16) && aligned(h_out, 16)) {
        // one decode step: blocks of 16 channels (G = 16 lanes each, N/16 states a
        // lane); measured 0.400 ms per d768x24 step at batch 8 against 0.414 with
        // 32-channel and 0.419 with 64-channel blocks
        const dim3 grid1((unsigned)(a.D / 16), (unsigned)B);
        switch (N) {
            case 16: hipLaunchKernelGGL((ssd_step_kernel<16, 1>), grid1, dim3(kMThreads), 0, st, a); break;
            case 32: hipLaunchKernelGGL((ssd_step_kernel<32, 2>), grid1, dim3(kMThreads), 0, st, a); break;
            default: hipLaunchKernelGGL((ssd_step_kernel<64, 4>), grid1, dim3(kMThreads), 0, st, a); break;
        }
        return hipGetLastError();
    }
    int G = N / 4;
    while (P % (kMThreads / G) != 0) G *= 2;  // P % 16 == 0, so G = 16 always fits
    const dim3 grid((unsigned)(a.D / (kMThreads / G)), (unsigned)B);
#define MI_SCASE(NN, GG)                                                                    \
    if (N == NN && G == GG) {                                                               \
        hipLaunchKernelGGL((ssd_scan_kernel<NN, GG>), grid, dim3(kMThreads), 0, st, a);     \
        return hipGetLastError();                                                           \
    }
    MI_SCASE(16, 4)
    MI_SCASE(16, 8)
    MI_SCASE(16, 16)
    MI_SCASE(32, 8)
    MI_SCASE(32, 16)
    MI_SCASE(64, 16)
#undef MI_SCASE
    return hipErrorInvalidValue;
}

// Used by mi_block_scan for N in {16, 32, 64}, D % 16 == 0 and 16-byte aligned rows.
hipError_t launch_model_scan(const int8_t *xs, const int8_t *dm, const int8_t *z, const int8_t *bsrc,
                             const int8_t *csrc, const int32_t *base, int8_t *yo, const int32_t *h_in, int32_t *h_out,
                             int64_t x_row, int64_t z_row, int64_t bc_row, int B, int L, int D, int N, int s_y,
                             hipStream_t st) {
    MScanArgs a{};
    a.xs = xs; a.dm = dm; a.z = z; a.bsrc = bsrc; a.csrc = csrc; a.base = base; a.yo = yo;
    a.h_in = h_in; a.h_out = h_out; a.x_row = x_row; a.z_row = z_row; a.bc_row = bc_row;
    a.B = B; a.L = L; a.D = D; a.s_y = s_y;
    // lanes per channel and block size, measured at d_inner 1536 x batch 8 x
    // L2048, N16 (ms per launch): G8/256 threads 0.333, G8/128 0.337, G4/64
    // 0.373, G4/256 0.369, G16/256 0.356, G4/128 0.531.  G4 (4 states a lane,
    // two DPP stages instead of three) wins once it still gives every SIMD
    // three waves, B * d_inner / 16 >= 3072 (L256, ms, G8 vs G4): B32 x 1536
    // 0.118 vs 0.113, B64 x 1536 0.219 vs 0.197, B32 x 4096 0.287 vs 0.262;
    // B16 x 1536 0.068 vs 0.074
    switch (N) {
        case 16:
            // 1024 < G8 waves <= 1536 (1.5 a SIMD at most): the mixed block of
            // 48 channels gives every SIMD one 2-state and one 1-state wave
            // when one block per CU (256 CUs) covers the batch.  d_inner 1536
            // x batch 8 x L2048: 0.317-0.325 ms (G8) -> 0.274-0.288 ms; the
            // staging pieces moved onto the 1-state waves: 0.310 ms
            if ((int64_t)B * D > 8192 && (int64_t)B * ((D + 47) / 48) <= 256)
                return launch_model_mix<16, 8, 16, 512>(a, st);
            return launch_model_n<16>((int64_t)B * D >= 3072 * 16 ? 4 : 8, 256, a, st);
        case 32: return launch_model_n<32>(8, 256, a, st);
        case 64: return launch_model_n<64>(16, 256, a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace mi
