// Fused decode-step stages of the integer Mamba block on gfx950 (spec
// mi-spec-2, rules 4.1-4.12 at one token per sequence).
//
// A decode step at small batch is bound by the chain of dependent kernels,
// not by bytes (the packed weights of the d768 x 24 model are 28.6 MB), so a
// layer runs as four kernels instead of seven:
//
//   norm_gemv      BitShiftNorm of the residual rows recomputed inside every
//                  block (rows <= 16, staged in LDS as int8), in_proj GEMV on
//                  MFMA, and for the x half the depthwise conv step + squareplus
//                  with the conv ring updated in place; the z half is stored.
//   (x_proj GEMV)  bitlinear.hip
//   dt_scan_step   dt_proj as a per-channel dot (v_dot4_i32_i8) fused with the
//                  decay clamp, dt, the scan state update, y = C.h, the gate and
//                  the requant of the out_proj input.
//   (out_proj GEMV + residual) bitlinear.hip
//
// The same norm_gemv (INT32 output, no conv) computes the lm_head logits.
#include "mi_mfma.hpp"

namespace mi {
namespace {

constexpr int kMaxRows = 16;    // tokens per norm_gemv block
constexpr int kMaxRowGroups = 4; // blocks along y: 16-token row groups of one launch
constexpr int kMaxNormK = 3072; // d_model limit of the LDS-staged rows
constexpr int kMaxXTiles = 16;  // x_proj outputs (dt_rank + 2*nstate) <= 256
constexpr int kMaxStatParts = 4096;  // row-statistics partials per row

struct NormGemvArgs {
    const int32_t *r;       // [M][K] residual, Q8
    const int64_t *row_stats;  // [M][stats_parts][2] (sum r, sum r^2) partials or null (computed here)
    int stats_parts;           // partials per row, summed here (1: full sums)
    const int16_t *gamma;   // [K]
    const uint32_t *w;      // [N][K/16] packed words
    void *out;              // INT32: [M][ldo]; INT8: [M][ldo] (z half written)
    int64_t ldo;
    int M, N, K, kw;
    int shift;
    // conv epilogue for features n < conv_d
    const int8_t *conv_w;   // [conv_d][4]
    const int32_t *conv_b;  // [conv_d]
    int8_t *conv_state;     // [M][3][conv_d]
    int8_t *xs;             // [M][conv_d]
    int conv_d;
    // x_proj partials of the x-blocks (optional): xpart[m][blk][nx] =
    // sum over the block's 16 channels c of w_x[n][c] * xs[m][c]
    const uint32_t *w_x;    // [nx][conv_d/16] words
    int nx;
    int32_t *xpart;
    // greedy-pick partials of the wide INT32 kernel (optional): keys[m][block]
    // = largest (logit << 32 | 0x7FFFFFFF - index) over the block's outputs
    int64_t *keys;
    // BitShiftNormV2's threshold table (the multi-head SSD block) instead of
    // MambaIntegerBlock's
    bool norm_v2;
};

__device__ __forceinline__ int norm_shift_args(const NormGemvArgs &g, int64_t s1, int64_t s2, int64_t *mu) {
    return g.norm_v2 ? norm_shift_tab<6, 2>(s1, s2, g.K, mu) : norm_shift_tab<8, 3>(s1, s2, g.K, mu);
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Normalized int8 rows (spec rule 4.1) of r[0..M) into LDS a[16][pitch].
// With row_stats: every thread normalizes 4-element groups of the flattened
// [M][K] rows; the loads of a whole chunk of groups are issued before the
// first wait, and threads 0..M-1 turn the row statistics into (mu, shift) in
// LDS meanwhile.  Without: one wave per row sums the row in one pass.
// Threads per row of the stats-driven staging: rows padded to a power of two
// Mp, TPR = 256/Mp threads each.
__device__ __forceinline__ int norm_tpr_log2(int M) { return M <= 1 ? 8 : M <= 2 ? 7 : M <= 4 ? 6 : M <= 8 ? 5 : 4; }
__device__ __forceinline__ int norm_tpr(int M) { return 1 << norm_tpr_log2(M); }

// Row statistics from stats_parts partials [M][P][2]: the RG = min(TPR, 64)
// lanes of a row's lane group (aligned to RG within the wave) each take the
// partials j0, j0 + RG, ... (a group's load covers contiguous bytes).  The
// first kStatLoads of them are loaded at kernel start, ahead of every other
// load and without a branch (no row_stats: a clamped dummy read of r), so
// the first wait for them does not hold back the loads issued after them;
// any further ones and the sum follow once the first chunk of row loads is
// in flight.  With P = 1 every lane reads its row's full sums.
constexpr int kStatLoads = 4;

struct StatParts {
    v2l v[kStatLoads];
};

// (16 lanes at most: the sum then stays inside a DPP row, with no cross-row
// shuffle through LDS; the 16 lanes of a row group's other halves repeat it)
__device__ __forceinline__ int stat_group(int M) { return min(norm_tpr(M), 16); }

__device__ __forceinline__ StatParts load_stat_parts(const NormGemvArgs &g, int mr) {
    const bool have = g.row_stats != nullptr;
    const int64_t *base = have ? g.row_stats : reinterpret_cast<const int64_t *>(g.r);
    const int P = have ? g.stats_parts : 1, row = have ? mr : 0;
    const int RG = stat_group(g.M), j0 = (int)threadIdx.x & (RG - 1);
    StatParts p;
#pragma unroll
    for (int u = 0; u < kStatLoads; ++u) {
        const int j = min(j0 + u * RG, P - 1);
        p.v[u] = *reinterpret_cast<const v2l *>(base + 2 * ((int64_t)row * P + j));
    }
    return p;
}

// (dpp_add64: v + the value of the lane a DPP control names, 64-bit, within
// rows of 16 lanes; mi_common.hpp)
// Sum over a lane group of 2^k lanes (aligned), every lane getting the total:
// quad swaps (xor 1, xor 2), then the half-row and row mirrors (lane i with
// 7 - i, then 15 - i: after the quad step each pairs with a lane of the other
// quad / other half-row), then xor shuffles across rows.
__device__ __forceinline__ int64_t group_sum64(int64_t v, int RG) {
    if (RG > 1) v = dpp_add64<0xB1>(v);   // quad_perm [1,0,3,2]
    if (RG > 2) v = dpp_add64<0x4E>(v);   // quad_perm [2,3,0,1]
    if (RG > 4) v = dpp_add64<0x141>(v);  // row_half_mirror
    if (RG > 8) v = dpp_add64<0x140>(v);  // row_mirror
    if (RG > 16) v += __shfl_xor(v, 16);
    if (RG > 32) v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ void sum_stat_parts(const NormGemvArgs &g, int mr, const StatParts &p, int64_t &s1,
                                               int64_t &s2) {
    if (g.stats_parts == 1) {
        s1 = p.v[0][0];
        s2 = p.v[0][1];
        return;
    }
    const int RG = stat_group(g.M), j0 = (int)threadIdx.x & (RG - 1);
    s1 = 0;
    s2 = 0;
#pragma unroll
    for (int u = 0; u < kStatLoads; ++u)
        if (j0 + u * RG < g.stats_parts) {
            s1 += p.v[u][0];
            s2 += p.v[u][1];
        }
    for (int j = j0 + kStatLoads * RG; j < g.stats_parts; j += RG) {
        const v2l v = *reinterpret_cast<const v2l *>(g.row_stats + 2 * ((int64_t)mr * g.stats_parts + j));
        s1 += v[0];
        s2 += v[1];
    }
    s1 = group_sum64(s1, RG);
    s2 = group_sum64(s2, RG);
}

// sp: the row statistics of this thread's row min(threadIdx.x / TPR, M - 1),
// loaded by the caller ahead of its other loads (used with row_stats).
__device__ void stage_norm_rows(const NormGemvArgs &g, int8_t *a, int pitch, const StatParts &sp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (g.row_stats) {
        // TPR threads per row, each with its row's (mu, shift) in registers
        // and groups tr, tr+TPR, ...
        const int lt = norm_tpr_log2(g.M), TPR = 1 << lt;   // shifts, not divides: ahead of the first loads
        const int m = (int)threadIdx.x >> lt, tr = (int)threadIdx.x & (TPR - 1);
        const int mr = min(m, g.M - 1);
        const int K4 = g.K / 4;
        constexpr int kC = 8;
        int4 rv[kC];
        uint2 gv[kC];
        const int32_t *row = g.r + (int64_t)mr * g.K;
        auto load_chunk = [&](int j0) {
#pragma unroll
            for (int c = 0; c < kC; ++c) {
                const int grp = min(tr + (j0 + c) * TPR, K4 - 1);
                rv[c] = *reinterpret_cast<const int4 *>(row + 4 * grp);
                gv[c] = *reinterpret_cast<const uint2 *>(g.gamma + 4 * grp);
            }
        };
        load_chunk(0);
        int64_t s1, s2;
        sum_stat_parts(g, mr, sp, s1, s2);
        int64_t mu64;
        const int sh = norm_shift_args(g, s1, s2, &mu64);
        const int32_t mu = (int32_t)mu64;
        const int64_t rnd = (int64_t)1 << (sh - 1);
        const int ngrp = (K4 + TPR - 1) >> lt;
        for (int j0 = 0; j0 < ngrp; j0 += kC) {
            if (j0 > 0) load_chunk(j0);
            // two groups (8 values) at a time: their 64-bit products are
            // independent chains written out one after another, every group
            // computed from its clamped load and stored unconditionally, a
            // group outside the rows into its row's padding bytes [K, K + 4)
            // that no MFMA reads (one basic block per pair: a branch per
            // group made each value wait on the one before it)
#pragma unroll
            for (int c0 = 0; c0 < kC; c0 += 2) {
                if (j0 + c0 >= ngrp) break;  // the same for the whole block
                int64_t p[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int c = c0 + (e >> 2), q = e & 3;
                    const int v = q == 0 ? rv[c].x : q == 1 ? rv[c].y : q == 2 ? rv[c].z : rv[c].w;
                    const uint32_t gw = q < 2 ? gv[c].x : gv[c].y;
                    const int gm = (int16_t)((q & 1) ? (gw >> 16) : (gw & 0xFFFF));
                    // |r - mu| < 2^24 and |gamma| < 2^15, so the rounded
                    // quotient (shift >= 9) fits 32 bits: the low word of
                    // the 64-bit shift is the exact value
                    p[e] = (int64_t)(v - mu) * gm + rnd;
                }
                uint32_t o[2] = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int32_t v = (int32_t)__builtin_amdgcn_alignbit((uint32_t)((uint64_t)p[e] >> 32),
                                                                         (uint32_t)p[e], (uint32_t)sh);
                    o[e >> 2] |= (uint32_t)(min(max(v, -127), 127) & 255) << (8 * (e & 3));
                }
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int grp = tr + (j0 + c0 + e) * TPR;
                    const int col = m < g.M && grp < K4 ? 4 * grp : g.K;   // m < 16 rows of a
                    *reinterpret_cast<uint32_t *>(&a[m * pitch + col]) = o[e];
                }
            }
        }
        return;
    }
    for (int m = wave; m < g.M; m += 4) {
        const int32_t *row = g.r + (int64_t)m * g.K;
        int64_t t1 = 0, t2 = 0;
        for (int i = lane; i < g.K; i += 64) {
            const int64_t v = row[i];
            t1 += v;
            t2 += v * v;
        }
        t1 = wave_sum64(t1);
        t2 = wave_sum64(t2);
        int64_t mu;
        const int sh = norm_shift_args(g, t1, t2, &mu);
        for (int i = 4 * lane; i < g.K; i += 256) {
            const int4 v = *reinterpret_cast<const int4 *>(row + i);
            const int vv[4] = {v.x, v.y, v.z, v.w};
            uint32_t o = 0;
            for (int q = 0; q < 4; ++q)
                o |= (uint32_t)((int)clamp64(rshr64((int64_t)(vv[q] - mu) * g.gamma[i + q], sh), -127, 127) & 255)
                     << (8 * q);
            *reinterpret_cast<uint32_t *>(&a[m * pitch + i]) = o;
        }
    }
}

// Two block shapes.  Narrow (WIDE = false): 16 output features per block, the
// 4 waves split K in 256-wide super-steps and reduce through LDS (in_proj:
// 192 blocks at d768).  Wide: 64 features per block, each wave owns 16 of them
// over the whole K, so the row normalization is shared by 4x more outputs
// (lm_head: 500 blocks instead of 2000).  Every global load that does not
// depend on the normalized rows (packed weights, conv ring, conv taps) is
// issued before the rows are staged, so its latency overlaps the staging.
constexpr int kMaxSuper = kMaxNormK / 256;

// The arguments of row group y (tokens [16y, 16y + 16)): every per-token
// pointer moves to the group's first row.
template <int KIND>
__device__ __forceinline__ NormGemvArgs row_group(const NormGemvArgs &g0, int y) {
    NormGemvArgs g = g0;
    const int64_t m0 = (int64_t)kMaxRows * y;
    g.M = min(kMaxRows, g0.M - (int)m0);
    g.r += m0 * g.K;
    if (g.row_stats) g.row_stats += m0 * g.stats_parts * 2;
    if (g.out) g.out = (char *)g.out + m0 * g.ldo * (KIND == MI_OUT_INT32 ? 4 : 1);
    if (g.conv_state) g.conv_state += m0 * 3 * g.conv_d;
    if (g.xs) g.xs += m0 * g.conv_d;
    if (g.xpart) g.xpart += m0 * (g.conv_d / 16) * g.nx;
    if (g.keys) g.keys += m0 * gridDim.x;
    return g;
}

template <int KIND, bool CONV, bool WIDE>
__global__ __launch_bounds__(256) void norm_gemv_kernel(NormGemvArgs g0) {
    const NormGemvArgs g = gridDim.y > 1 ? row_group<KIND>(g0, blockIdx.y) : g0;
    // narrow blocks: the dispatcher deals consecutive block ids to the 8 XCDs
    // in turn; renumbering gives each XCD a contiguous run of features, so the
    // conv taps, ring bytes and x_proj words its blocks share sit in one L2
    // (decode in_proj stage at d768, batch 8: 5.01 -> 4.80 us)
    const int blk = !WIDE && (gridDim.x & 7) == 0 ? (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3)
                                                  : (int)blockIdx.x;
    extern __shared__ __align__(16) int8_t smem[];
    const int pitch = g.K + 16;                       // conflict-free b128 row reads
    int8_t *a = smem;                                 // [16][pitch]
    v4i *red = reinterpret_cast<v4i *>(smem + kMaxRows * pitch);  // [4][64]

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int l16 = lane & 15, lq = lane >> 4;
    // the row statistics of this thread's staging row, before any other load
    const StatParts sp = load_stat_parts(g, min(tid >> norm_tpr_log2(g.M), g.M - 1));
    const int n0 = WIDE ? blockIdx.x * 64 + wave * 16 : blk * 16;
    const int n = n0 + l16;
    const int nsuper = (g.kw + 15) / 16;
    constexpr int kPer = WIDE ? kMaxSuper : (kMaxSuper + 3) / 4;
    const int s_first = WIDE ? 0 : wave, s_step = WIDE ? 1 : 4;

    // packed weights: one 16-byte load (4 words) per lane and super-step,
    // from a clamped row (its outputs are not stored); words past K meet
    // zero activations
    uint32_t wv[kPer][4];
    {
        const uint32_t *wrow = g.w + (int64_t)min(n, g.N - 1) * g.kw;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            if (s_first + i * s_step < nsuper) {
                const int w0 = min(16 * (s_first + i * s_step) + 4 * lq, g.kw - 4);
                const uint4 q4 = *reinterpret_cast<const uint4 *>(wrow + w0);
                wv[i][0] = q4.x; wv[i][1] = q4.y; wv[i][2] = q4.z; wv[i][3] = q4.w;
            }
        }
    }
    // conv operands of this lane's epilogue (token l16, features nf..nf+3)
    const int m = l16;
    const int nf = n0 + 4 * lq;
    const bool epi = (WIDE || wave == 0) && m < g.M && nf < g.N;
    const bool conv = CONV && WIDE && epi && nf < g.conv_d;
    uint32_t cs0 = 0, cs1 = 0, cs2 = 0, cw[4] = {0, 0, 0, 0};
    int32_t cb[4] = {0, 0, 0, 0};
    // narrow conv kernel: every thread owns one output (token l16, feature
    // n0 + 4lq + wave) of an x-block and prefetches that channel's operands
    const bool xblk = CONV && !WIDE && n0 < g.conv_d;
    int ecs0 = 0, ecs1 = 0, ecs2 = 0, ecb = 0;
    uint32_t ecw = 0;
    if (xblk) {
        const int ch = nf + wave;  // < conv_d: conv_d % 16 == 0
        const int8_t *st = g.conv_state + (int64_t)min(m, g.M - 1) * 3 * g.conv_d + ch;
        ecs0 = st[0];
        ecs1 = st[g.conv_d];
        ecs2 = st[2 * g.conv_d];
        ecw = *reinterpret_cast<const uint32_t *>(g.conv_w + (int64_t)ch * 4);
        ecb = g.conv_b[ch];
    }
    if (conv) {
        const int8_t *st = g.conv_state + (int64_t)m * 3 * g.conv_d;
        cs0 = *reinterpret_cast<const uint32_t *>(st + nf);
        cs1 = *reinterpret_cast<const uint32_t *>(st + g.conv_d + nf);
        cs2 = *reinterpret_cast<const uint32_t *>(st + 2 * g.conv_d + nf);
        for (int r = 0; r < 4; ++r) {
            cw[r] = *reinterpret_cast<const uint32_t *>(g.conv_w + (int64_t)(nf + r) * 4);
            cb[r] = g.conv_b[nf + r];
        }
    }

    // x_proj words of this block's 16 channels (x-blocks; wave w takes the 16-row tiles w, w+4, ...)
    const bool xpart = CONV && !WIDE && g.xpart != nullptr && n0 < g.conv_d;
    uint32_t wx[kMaxXTiles / 4];
    if (xpart) {
        const int xkw = g.conv_d / 16;
#pragma unroll
        for (int u = 0; u < kMaxXTiles / 4; ++u) {
            const int t = 4 * u + wave;
            wx[u] = 16 * t < g.nx ? g.w_x[(int64_t)min(16 * t + l16, g.nx - 1) * xkw + n0 / 16] : 0u;
        }
    }

    stage_norm_rows(g, a, pitch, sp);
    __syncthreads();

    v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int sidx = s_first + i * s_step;
        if (sidx < nsuper) {
            const int w0 = 16 * sidx + 4 * lq;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = 16 * (w0 + j);
                v4i fa = v4i{0, 0, 0, 0};
                if (k < g.K) fa = *reinterpret_cast<const v4i *>(&a[l16 * pitch + k]);
                acc = mfma_i8(unpack16(wv[i][j]), fa, acc);
            }
        }
    }
    if constexpr (CONV && !WIDE) {
        // all four waves finish the block: thread (wave, lane) takes output
        // (token l16, feature n0 + 4lq + wave), the MFMA result register
        // `wave` summed over the four waves' partial products
        red[wave * 64 + lane] = acc;
        __syncthreads();
        const int32_t v = red[lane][wave] + red[64 + lane][wave] + red[128 + lane][wave] + red[192 + lane][wave];
        const int q = clamp32(rshr32(v, g.shift), -127, 127);
        const int fe = nf + wave;
        const bool ok = m < g.M && fe < g.N;
        if (!xblk) {
            if (ok) reinterpret_cast<int8_t *>(g.out)[(int64_t)m * g.ldo + fe] = (int8_t)q;  // z half
            return;
        }
        // depthwise conv step (conv1d_step.cu:30-57) + squareplus of one channel
        int xsv = 0;
        if (ok) {
            const int32_t c = ecb + (int)(int8_t)ecw * ecs0 + (int)(int8_t)(ecw >> 8) * ecs1 +
                              (int)(int8_t)(ecw >> 16) * ecs2 + (int)(int8_t)(ecw >> 24) * q;
            xsv = sqp_q(c);
            g.xs[(int64_t)m * g.conv_d + fe] = (int8_t)xsv;
            int8_t *st = g.conv_state + (int64_t)m * 3 * g.conv_d + fe;
            st[0] = (int8_t)ecs1;
            st[g.conv_d] = (int8_t)ecs2;
            st[2 * g.conv_d] = (int8_t)q;
        }
        if (!xpart) return;
        // the block's x_proj partial: one MFMA per 16 x_proj rows with K = the
        // block's 16 channels (lane group lq carries channels 4lq..4lq+3 in
        // its first dword, the other k slots are zero)
        __shared__ uint32_t s_xs[16][4];
        reinterpret_cast<int8_t *>(&s_xs[m][lq])[wave] = (int8_t)xsv;
        __syncthreads();
        const v4i fb = v4i{(int)s_xs[l16][lq], 0, 0, 0};
        const uint32_t lut = 0xFFFE0100u;
        const int nblk = g.conv_d / 16;
        int32_t *dst = g.xpart + ((int64_t)m * nblk + blk) * g.nx;
        // every product first, then the stores back to back (a store between
        // two MFMAs would make the next wait on its completion)
        v4i d[kMaxXTiles / 4];
#pragma unroll
        for (int u = 0; u < kMaxXTiles / 4; ++u) {
            const int t = 4 * u + wave;
            if (16 * t < g.nx) {
                const v4i fa = v4i{(int)__builtin_amdgcn_perm(lut, lut, (wx[u] >> (2 * lq)) & 0x03030303u), 0, 0, 0};
                d[u] = mfma_i8(fa, fb, v4i{0, 0, 0, 0});
            }
        }
        // lane (token l16, group lq) holds rows 16t + 4lq + r
        if (m < g.M) {
#pragma unroll
            for (int u = 0; u < kMaxXTiles / 4; ++u) {
                const int t = 4 * u + wave;
                const int row = 16 * t + 4 * lq;
                if (16 * t < g.nx) {
                    if ((g.nx & 3) == 0 && row + 3 < g.nx) {
                        *reinterpret_cast<v4i *>(dst + row) = d[u];
                    } else {
                        for (int r = 0; r < 4; ++r)
                            if (row + r < g.nx) dst[row + r] = d[u][r];
                    }
                }
            }
        }
        return;
    }
    if (!WIDE) {
        if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = acc + red[lane] + red[64 + lane] + red[128 + lane];
    }
    if constexpr (WIDE && KIND == MI_OUT_INT32) {
        if (g.keys) {
            // the larger logit wins; among equal logits the smaller index
            __shared__ int64_t s_key[4][16];
            int64_t best = INT64_MIN;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (nf + r < g.N)
                    best = max(best, (int64_t)(((uint64_t)(int64_t)acc[r] << 32) | (uint32_t)(0x7FFFFFFF - (nf + r))));
            best = max(best, (int64_t)__shfl_xor(best, 16));
            best = max(best, (int64_t)__shfl_xor(best, 32));
            if (lq == 0) s_key[wave][l16] = best;
            __syncthreads();
            if (tid < g.M)
                g.keys[(int64_t)tid * gridDim.x + blockIdx.x] =
                    max(max(s_key[0][tid], s_key[1][tid]), max(s_key[2][tid], s_key[3][tid]));
            if (g.out == nullptr) return;
        }
    }
    if (!epi) return;
    if constexpr (KIND == MI_OUT_INT32) {
        int32_t *o = (int32_t *)g.out + (int64_t)m * g.ldo + nf;
        for (int r = 0; r < 4 && nf + r < g.N; ++r) o[r] = acc[r];
    } else {
        int v[4];
        for (int r = 0; r < 4; ++r) v[r] = clamp32(rshr32(acc[r], g.shift), -127, 127);
        if (conv) {
            // depthwise conv step (conv1d_step.cu:30-57) + squareplus on 4 channels
            uint32_t xsw = 0, cur = 0;
            for (int r = 0; r < 4; ++r) {
                int32_t c = cb[r];
                c += (int)(int8_t)(cw[r]) * (int)(int8_t)(cs0 >> (8 * r));
                c += (int)(int8_t)(cw[r] >> 8) * (int)(int8_t)(cs1 >> (8 * r));
                c += (int)(int8_t)(cw[r] >> 16) * (int)(int8_t)(cs2 >> (8 * r));
                c += (int)(int8_t)(cw[r] >> 24) * v[r];
                xsw |= (uint32_t)(sqp_q(c) & 255) << (8 * r);
                cur |= (uint32_t)(v[r] & 255) << (8 * r);
            }
            int8_t *st = g.conv_state + (int64_t)m * 3 * g.conv_d;
            *reinterpret_cast<uint32_t *>(g.xs + (int64_t)m * g.conv_d + nf) = xsw;
            *reinterpret_cast<uint32_t *>(st + nf) = cs1;
            *reinterpret_cast<uint32_t *>(st + g.conv_d + nf) = cs2;
            *reinterpret_cast<uint32_t *>(st + 2 * g.conv_d + nf) = cur;
        } else {
            int8_t *o = (int8_t *)g.out + (int64_t)m * g.ldo + nf;
            for (int r = 0; r < 4 && nf + r < g.N; ++r) o[r] = (int8_t)v[r];
        }
    }
}

// ------------------------------------------------------------ dt + scan step
struct DtScanArgs {
    const int8_t *xp;       // [M][xp_stride]: dt_raw at [0,R), B at [R,R+N), C at [R+N,R+2N)
    int64_t xp_stride;
    const uint32_t *w_x;    // fused x_proj: [R+2N][D/16] words (xp unused)
    int s_x;
    bool x_c16;             // w_x rows are whole 16-word chunks, 16-byte aligned
    const int32_t *xpart;   // x_proj partials [M][nblk][R+2N] (XNT < 0)
    int nblk;
    int R;
    const uint32_t *w_dt;   // [D][R/16] words
    int s_dt;
    const int8_t *xs;       // [M][D]
    const int8_t *z;        // [M][z_stride] (already offset to the z columns)
    int64_t z_stride;
    const int32_t *base;    // [D][N]
    int k, s_y;
    int32_t *h;             // [M][D][N] in place
    int8_t *yo;             // [M][D]
    int M, D, N;
};

constexpr int kMaxR = 256;
__constant__ StepTables kStepTables = make_step_tables();
constexpr int kMaxN = 64;
constexpr int kTokMaxParts = 4;  // x_proj partials per token that dt_scan_tok_kernel sums itself

// Thread quad per channel: lane g of the quad keeps states g, g+4, g+8, ...;
// every lane computes the channel's dt_proj dot (48-wide at d768), the quad
// sums y with two DPP adds, lane 0 gates and writes.
// x_proj outputs of token m (the block's own copy): 16x16x64 MFMA with the
// ternary rows as the A operand and the token in column 0 of B (the other
// columns zero).  Each of the 16 lane groups (4 waves x 4 k-groups) owns a
// contiguous run of packed words, so every lane reads 8-byte pairs of words
// of its row and all loads of a chunk are issued before the first MFMA; the
// word -> k-group assignment is the same for A and B, so the dot products are
// unchanged.  Column-0 lanes leave per-wave partial sums in s_xacc.
template <int NT>
__device__ __forceinline__ void xproj_token(const DtScanArgs &g, int m, int32_t (*s_xacc)[16 * kMaxXTiles]) {
    constexpr int CW = (64 / NT) >= 8 ? 8 : ((64 / NT) & ~1);
    static_assert(CW >= 2 && CW % 2 == 0, "chunk of word pairs");
    const int lane = threadIdx.x & 63, wave = wave_id(), l16 = lane & 15, lq = lane >> 4;
    const int NX = g.R + 2 * g.N;
    const int kwx = g.D / 16;               // even: d_inner % 32 == 0
    const int wpg = 2 * ((kwx + 31) / 32);  // words per lane group, even
    const int w0 = (wave * 4 + lq) * wpg;
    const int w1 = min(w0 + wpg, kwx);
    const int8_t *xrow = g.xs + (int64_t)m * g.D;
    v4i acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
    // the trip count is the same for every lane (MFMA reads all 64 lanes, so
    // no lane may skip it); words past a group's run load as zeros
    for (int c0 = 0; c0 < wpg; c0 += CW) {
        // every load is unconditional, from a clamped in-bounds address (a
        // divergent load would make the compiler wait on it before the next
        // one): rows past NX feed result rows nobody reads, and words past
        // the group's run meet a zero B operand
        uint2 wv[NT][CW / 2];
        v4i xv[CW];
#pragma unroll
        for (int p = 0; p < CW / 2; ++p) {
            const int wc = min(w0 + c0 + 2 * p, kwx - 2);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int n = min(16 * t + l16, NX - 1);
                wv[t][p] = *reinterpret_cast<const uint2 *>(g.w_x + (int64_t)n * kwx + wc);
            }
            xv[2 * p] = *reinterpret_cast<const v4i *>(xrow + 16 * wc);
            xv[2 * p + 1] = *reinterpret_cast<const v4i *>(xrow + 16 * wc + 16);
        }
#pragma unroll
        for (int p = 0; p < CW / 2; ++p) {
            const bool xa = l16 == 0 && w0 + c0 + 2 * p < w1;
            const v4i f0 = xa ? xv[2 * p] : v4i{0, 0, 0, 0};
            const v4i f1 = xa ? xv[2 * p + 1] : v4i{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc[t] = mfma_i8(unpack16(wv[t][p].x), f0, acc[t]);
                acc[t] = mfma_i8(unpack16(wv[t][p].y), f1, acc[t]);
            }
        }
    }
    // column-0 lanes (l16 == 0) hold features 16t + 4lq + r
    if (l16 == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) s_xacc[wave][16 * t + 4 * lq + r] = acc[t][r];
    }
}

// Coalesced variant for d_inner % 256 == 0 (the packed row is a whole number
// of 16-word chunks): wave v takes chunks v, v+4, ...; in a chunk, lane
// (l16, lq) reads words [4lq, 4lq+4) of row 16t+l16 as one 16-byte load, so
// one load instruction covers 64 contiguous bytes of each of 16 rows, and the
// four words feed four MFMA k-steps.  Two chunks' loads are in flight at once.
template <int NT>
__device__ __forceinline__ void xproj_token_c16(const DtScanArgs &g, int m, int32_t (*s_xacc)[16 * kMaxXTiles]) {
    const int lane = threadIdx.x & 63, wave = wave_id(), l16 = lane & 15, lq = lane >> 4;
    const int NX = g.R + 2 * g.N;
    const int kwx = g.D / 16;
    const int nchunk = kwx / 16;
    const int8_t *xrow = g.xs + (int64_t)m * g.D;
    v4i acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
    for (int c0 = wave; c0 < nchunk; c0 += 8) {
        v4i wv[2][NT];
        v4i xv[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            // a second chunk past the end re-reads the first (in bounds) and meets a zero B operand
            const int c = c0 + 4 * u < nchunk ? c0 + 4 * u : c0;
            const int w = 16 * c + 4 * lq;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int n = min(16 * t + l16, NX - 1);
                wv[u][t] = *reinterpret_cast<const v4i *>(g.w_x + (int64_t)n * kwx + w);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[u][j] = *reinterpret_cast<const v4i *>(xrow + 16 * (w + j));
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const bool xa = l16 == 0 && c0 + 4 * u < nchunk;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v4i f = xa ? xv[u][j] : v4i{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_i8(unpack16((uint32_t)wv[u][t][j]), f, acc[t]);
            }
        }
    }
    if (l16 == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) s_xacc[wave][16 * t + 4 * lq + r] = acc[t][r];
    }
}

// XNT > 0: the block first computes the x_proj outputs of its token itself
// (XNT tiles of 16 features, the x_proj weights come from L2), so the
// separate x_proj GEMV kernel and its launch leave the decode chain.
// NPL > 0 (nstate == 4*NPL): lane q of a channel owns the contiguous states
// [q*NPL, q*NPL+NPL), read and written as int4; NPL == 0: lane q owns states
// q, q+4, ... (any nstate <= 64).  Every load is issued unconditionally from
// an in-bounds address before the first wait.
// S24 (NPL = 4, decay_shift 15): the state update in 24-bit multiplies
// (update16, as in dt_scan_tok_kernel) and y as two int32 partial sums.
template <int XNT, int NPL, bool S24 = false>
__global__ __launch_bounds__(256) void dt_scan_step_kernel(DtScanArgs g) {
    __shared__ __align__(16) int8_t s_dt[kMaxR];
    __shared__ int8_t s_bc[2 * kMaxN];
    __shared__ int32_t s_xacc[XNT ? 4 : 1][XNT ? 16 * kMaxXTiles : 1];  // XNT < 0: row 0 only
    __shared__ int32_t s_dtq[41];    // dt_q16(dm) for dm in [-20, 20]
    __shared__ int32_t s_gate[256];  // gate_q15(z) for z in [-128, 127] (the block has 256 threads)
    // table entries load with the other independent loads; they reach LDS
    // just before the first barrier, after every other load has been issued
    const int32_t tab_dt = kStepTables.dtq[min((int)threadIdx.x, 40)];
    const int32_t tab_gate = kStepTables.gate[threadIdx.x];
    auto stage_tables = [&]() {
        if (threadIdx.x < 41) s_dtq[threadIdx.x] = tab_dt;
        s_gate[threadIdx.x] = tab_gate;
    };
    constexpr int kPerLane = NPL > 0 ? NPL : kMaxN / 4;
    // (placing a token's blocks on one XCD, so its x_proj partials are read
    // into one L2, measured 3.65 -> 3.73 us at batch 8: the renumbering's
    // division costs more than the L2 misses it saves)
    const int m = blockIdx.y;
    const int q = threadIdx.x & 3;
    const int d = blockIdx.x * 64 + (threadIdx.x >> 2);
    const bool active = d < g.D;
    const int dd = active ? d : g.D - 1;
    // loads that do not depend on the staged row: ternary dt_proj words, state, decays, xs, z
    // the dt_proj dot of a channel is split over its 4 lanes: lane q takes
    // the packed words q, q+4, ... (clamped loads; words past kw are skipped)
    const int kw = g.R / 16;
    uint32_t wdt[kMaxR / 64];
#pragma unroll
    for (int i = 0; i < kMaxR / 64; ++i)  // unconditional (kw >= 1): words past kw are never used
        wdt[i] = g.w_dt[(int64_t)dd * kw + min(q + 4 * i, kw - 1)];
    int32_t *hp = g.h + ((int64_t)m * g.D + dd) * g.N;
    const int32_t *bp = g.base + (int64_t)dd * g.N;
    int32_t hv[kPerLane], bv[kPerLane];
    if constexpr (NPL > 0) {
#pragma unroll
        for (int c = 0; c < NPL / 4; ++c) {
            // the state is read and written once a step: non-temporal, so its
            // stream does not displace the weights in L2 (0.2950 -> 0.2943 ms
            // per d768 x 24 step at batch 8)
            const v4i h4 = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(hp + q * NPL + 4 * c));
            const int4 b4 = *reinterpret_cast<const int4 *>(bp + q * NPL + 4 * c);
            hv[4 * c] = h4[0]; hv[4 * c + 1] = h4[1]; hv[4 * c + 2] = h4[2]; hv[4 * c + 3] = h4[3];
            bv[4 * c] = b4.x; bv[4 * c + 1] = b4.y; bv[4 * c + 2] = b4.z; bv[4 * c + 3] = b4.w;
        }
    } else {
        const int nq = (g.N + 3) >> 2;  // same for every lane
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) {
            if (i < nq) {
                const int n = min(q + 4 * i, g.N - 1);
                hv[i] = hp[n];
                bv[i] = bp[n];
            } else {
                hv[i] = 0;
                bv[i] = 0;
            }
        }
    }
    const int xsv = g.xs[(int64_t)m * g.D + dd];
    const int zv = g.z[(int64_t)m * g.z_stride + dd];

    if constexpr (XNT < 0) {
        // x_proj from the producer's per-block partials: thread (sub, n) sums
        // blocks sub, sub+S, ... of output n (32 loads in flight), the S
        // sub-sums meet in LDS
        const int NX = g.R + 2 * g.N;
        const int S = max(1, 256 / NX);
        const int sub = threadIdx.x / NX;
        const int n = (int)threadIdx.x - sub * NX;
        if (sub < S) {
            const int nb = g.nblk;
            const int32_t *pp = g.xpart + (int64_t)m * nb * NX + n;
            int32_t sum = 0;
            for (int b0 = sub; b0 < nb; b0 += 32 * S) {
                int32_t v[32];
#pragma unroll
                for (int u = 0; u < 32; ++u) v[u] = pp[(int64_t)min(b0 + u * S, nb - 1) * NX];
#pragma unroll
                for (int u = 0; u < 32; ++u) sum += b0 + u * S < nb ? v[u] : 0;
            }
            s_xacc[0][sub * NX + n] = sum;
        }
        stage_tables();
        __syncthreads();
        for (int i = threadIdx.x; i < NX; i += 256) {
            int v = 0;
            for (int k = 0; k < S; ++k) v += s_xacc[0][k * NX + i];
            const int8_t q8 = (int8_t)clamp32(rshr32(v, g.s_x), -127, 127);
            if (i < g.R) s_dt[i] = q8;
            else s_bc[i - g.R] = q8;
        }
    } else if constexpr (XNT > 0) {
        if (g.x_c16) xproj_token_c16<(XNT > 0 ? XNT : 1)>(g, m, s_xacc);
        else xproj_token<(XNT > 0 ? XNT : 1)>(g, m, s_xacc);
        stage_tables();
        __syncthreads();
        const int NX = g.R + 2 * g.N;
        for (int i = threadIdx.x; i < NX; i += 256) {
            const int v = s_xacc[0][i] + s_xacc[1][i] + s_xacc[2][i] + s_xacc[3][i];
            const int8_t q8 = (int8_t)clamp32(rshr32(v, g.s_x), -127, 127);
            if (i < g.R) s_dt[i] = q8;
            else s_bc[i - g.R] = q8;
        }
    } else {
        const int8_t *row = g.xp + (int64_t)m * g.xp_stride;
        for (int i = threadIdx.x; i < g.R; i += 256) s_dt[i] = row[i];
        for (int i = threadIdx.x; i < 2 * g.N; i += 256) s_bc[i] = row[g.R + i];
    }
    if constexpr (XNT == 0) stage_tables();
    __syncthreads();

    int acc = 0;
#pragma unroll
    for (int i = 0; i < kMaxR / 64; ++i) {
        const int w = q + 4 * i;
        if (w < kw) {
            const v4i wt = unpack16(wdt[i]);
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_sdot4(wt[j], *reinterpret_cast<const int *>(&s_dt[16 * w + 4 * j]), acc, false);
        }
    }
    acc = quad_sum(acc);
    const int dm = clamp32(rshr32(acc, g.s_dt), -20, 20);
    const int64_t xd = rshr64((int64_t)xsv * s_dtq[dm + 20], 10);
    int64_t y = 0;
    if constexpr (NPL > 0) {
        int32_t hn[NPL];
        if constexpr (S24) {
            // |x * dt| <= 127 * 6554: the rounded shift is exact in 32 bits;
            // the base is clamped to [-21, 32021] first (with |dm| <= 20 the
            // decay clamp(base + dm, 0, 32000) is unchanged) and doubled
            static_assert(NPL == 4, "S24 takes 4 states a lane");
            const int xd32 = (xsv * s_dtq[dm + 20] + 512) >> 10;
            int yh = 0, yl = 0;
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int n = q * NPL + i;
                const int n2 = min(max(2 * clamp32(bv[i], -21, 32021) + 2 * dm, 0), 64000);
                hn[i] = hv[i];
                update16(hn[i], n2, __mul24((int)s_bc[n], xd32), (int)s_bc[g.N + n], yh, yl);
            }
            y = (int64_t)quad_sum(yh) * 65536 + quad_sum(yl);
        } else {
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int n = q * NPL + i;
                const int64_t nt = clamp64((int64_t)bv[i] + dm, 0, 32000);
                hn[i] = sat32_64((((int64_t)hv[i] * nt) >> g.k) + (int64_t)s_bc[n] * xd);
                y += (int64_t)s_bc[g.N + n] * hn[i];
            }
            y = quad_sum64(y);
        }
        if (active) {
#pragma unroll
            for (int c = 0; c < NPL / 4; ++c)
                __builtin_nontemporal_store(v4i{hn[4 * c], hn[4 * c + 1], hn[4 * c + 2], hn[4 * c + 3]},
                                            reinterpret_cast<v4i *>(hp + q * NPL + 4 * c));
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) {
            const int n = q + 4 * i;
            if (active && n < g.N) {
                const int64_t nt = clamp64((int64_t)bv[i] + dm, 0, 32000);
                const int32_t hn = sat32_64((((int64_t)hv[i] * nt) >> g.k) + (int64_t)s_bc[n] * xd);
                hp[n] = hn;
                y += (int64_t)s_bc[g.N + n] * hn;
            }
        }
        y = quad_sum64(y);
    }
    if (active && q == 0) {
        const int64_t yg = ((int64_t)sat32_64(y) * s_gate[zv + 128]) >> 15;
        g.yo[(int64_t)m * g.D + d] = (int8_t)clamp64(rshr64(yg, g.s_y), -127, 127);
    }
}

// mi_dt_scan_step for nstate 16 with TPB tokens per block (same 64 channels):
// the dt_proj words (unpacked once), the decays and the tables serve all TPB
// tokens, and each lane keeps TPB int4 state vectors in flight.  Lane q of a
// channel owns states 4q..4q+3, as in dt_scan_step_kernel<0, 4>.
// XP: the x_proj rows arrive as nblk <= kTokMaxParts int32 partial sums per
// token (mi_xpart_dt_scan_step), summed and requantised while staging.
// S24 (decay_shift 15): the state update in 24-bit multiplies (update16:
// h read as H = h >> 16 and L = h & 0xffff, n2 = 2 * nt <= 64000, so
// floor(h * nt / 2^15) = H * n2 + floor(L * n2 / 2^16) exactly); B * xd fits
// 32 bits (|xd| <= 813), so the sum saturates with one clamped add; y = C . h
// accumulates C * H and C * L in two int32 sums (each < 2^29 over a channel's
// 16 states).  Without S24 the same rules run in 64-bit arithmetic.
template <int TPB, bool XP, bool S24>
__global__ __launch_bounds__(256) void dt_scan_tok_kernel(DtScanArgs g) {
    __shared__ __align__(16) int8_t s_dt[TPB][kMaxR];
    __shared__ __align__(16) int8_t s_bc[TPB][32];
    __shared__ int32_t s_dtq[41];
    __shared__ int32_t s_gate[256];
    const int32_t tab_dt = kStepTables.dtq[min((int)threadIdx.x, 40)];
    const int32_t tab_gate = kStepTables.gate[threadIdx.x];
    const int m0 = blockIdx.y * TPB;
    const int q = threadIdx.x & 3;
    const int d = blockIdx.x * 64 + (threadIdx.x >> 2);
    const bool active = d < g.D;
    const int dd = active ? d : g.D - 1;
    const int kw = g.R / 16;
    uint32_t wdt[kMaxR / 64];
#pragma unroll
    for (int i = 0; i < kMaxR / 64; ++i)  // unconditional (kw >= 1): words past kw are never used
        wdt[i] = g.w_dt[(int64_t)dd * kw + min(q + 4 * i, kw - 1)];
    const int4 b4 = *reinterpret_cast<const int4 *>(g.base + (int64_t)dd * 16 + 4 * q);
    // S24: 2 * base, the base first clamped to [-21, 32021] (with |dm| <= 20,
    // clamp(base + dm, 0, 32000) is unchanged and the doubling cannot overflow)
    const int b2[4] = {2 * clamp32(b4.x, -21, 32021), 2 * clamp32(b4.y, -21, 32021), 2 * clamp32(b4.z, -21, 32021),
                       2 * clamp32(b4.w, -21, 32021)};
    v4i h4[TPB];   // streamed: the whole state is read and written once per step
    int xsv[TPB], zv[TPB];
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        const int mt = min(m0 + t, g.M - 1);
        h4[t] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(g.h + ((int64_t)mt * g.D + dd) * 16 + 4 * q));
        xsv[t] = g.xs[(int64_t)mt * g.D + dd];
        zv[t] = g.z[(int64_t)mt * g.z_stride + dd];
    }
    // the TPB x_proj rows (dt_raw, B, C): every byte load issued before the
    // first wait, from clamped in-bounds positions; staged into LDS below
    // (XP: thread i < TPB*nxr/4 loads outputs 4i..4i+3 of every partial as
    // 16-byte vectors; nxr is a multiple of 16, so a group never straddles
    // two tokens or the dt_raw / B boundary)
    const int nxr = g.R + 32;
    constexpr int kXpLoads = XP ? 1 : (TPB * (kMaxR + 32) + 255) / 256;
    static_assert(!XP || TPB * (kMaxR + 32) / 4 <= 256, "one 4-output group per thread");
    int8_t xpv[kXpLoads];
    v4i xq4[XP ? kTokMaxParts : 1];
    if constexpr (XP) {
        const int gi = min((int)threadIdx.x, TPB * nxr / 4 - 1);
        const int t = 4 * gi / nxr, c = 4 * gi - t * nxr;
        const int mt = min(m0 + t, g.M - 1);
#pragma unroll
        for (int b = 0; b < kTokMaxParts; ++b)
            xq4[b] = *reinterpret_cast<const v4i *>(g.xpart + ((int64_t)mt * g.nblk + min(b, g.nblk - 1)) * nxr + c);
    } else {
#pragma unroll
        for (int u = 0; u < kXpLoads; ++u) {
            const int i = min((int)threadIdx.x + 256 * u, TPB * nxr - 1);
            const int t = i / nxr, c = i - t * nxr;
            xpv[u] = g.xp[(int64_t)min(m0 + t, g.M - 1) * g.xp_stride + c];
        }
    }
    v4i wt[kMaxR / 64];
#pragma unroll
    for (int i = 0; i < kMaxR / 64; ++i) wt[i] = unpack16(wdt[i]);  // words past kw are skipped below
    if constexpr (XP) {
        const int gi = (int)threadIdx.x;
        if (gi < TPB * nxr / 4) {
            const int t = 4 * gi / nxr, c = 4 * gi - t * nxr;
            v4i sum = xq4[0];
#pragma unroll
            for (int b = 1; b < kTokMaxParts; ++b)
                if (b < g.nblk) sum += xq4[b];
            uint32_t q = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) q |= (uint32_t)(clamp32(rshr32(sum[r], g.s_x), -127, 127) & 255) << (8 * r);
            *reinterpret_cast<uint32_t *>(c < g.R ? &s_dt[t][c] : &s_bc[t][c - g.R]) = q;
        }
    } else {
#pragma unroll
        for (int u = 0; u < kXpLoads; ++u) {
            const int i = (int)threadIdx.x + 256 * u;
            if (i < TPB * nxr) {
                const int t = i / nxr, c = i - t * nxr;
                if (c < g.R) s_dt[t][c] = xpv[u];
                else s_bc[t][c - g.R] = xpv[u];
            }
        }
    }
    if (threadIdx.x < 41) s_dtq[threadIdx.x] = tab_dt;
    s_gate[threadIdx.x] = tab_gate;
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        const int m = m0 + t;
        int acc = 0;
#pragma unroll
        for (int i = 0; i < kMaxR / 64; ++i) {
            const int w = q + 4 * i;
            if (w < kw) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = __builtin_amdgcn_sdot4(wt[i][j], *reinterpret_cast<const int *>(&s_dt[t][16 * w + 4 * j]),
                                                 acc, false);
            }
        }
        acc = quad_sum(acc);
        const int dm = clamp32(rshr32(acc, g.s_dt), -20, 20);
        const int hv[4] = {h4[t][0], h4[t][1], h4[t][2], h4[t][3]};
        const int bv[4] = {b4.x, b4.y, b4.z, b4.w};
        int32_t hn[4];
        int64_t y = 0;
        if constexpr (S24) {
            // |x * dt| <= 127 * 6554: the rounded shift is exact in 32 bits
            const int xd = (xsv[t] * s_dtq[dm + 20] + 512) >> 10;
            const int bw = *reinterpret_cast<const int *>(&s_bc[t][4 * q]);
            const int cw = *reinterpret_cast<const int *>(&s_bc[t][16 + 4 * q]);
            int yh = 0, yl = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n2 = min(max(b2[i] + 2 * dm, 0), 64000);
                const int bn = (bw << (24 - 8 * i)) >> 24, cn = (cw << (24 - 8 * i)) >> 24;
                hn[i] = hv[i];
                update16(hn[i], n2, __mul24(bn, xd), cn, yh, yl);
            }
            y = (int64_t)quad_sum(yh) * 65536 + quad_sum(yl);
        } else {
            const int64_t xd = rshr64((int64_t)xsv[t] * s_dtq[dm + 20], 10);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = 4 * q + i;
                const int64_t nt = clamp64((int64_t)bv[i] + dm, 0, 32000);
                hn[i] = sat32_64((((int64_t)hv[i] * nt) >> g.k) + (int64_t)s_bc[t][n] * xd);
                y += (int64_t)s_bc[t][16 + n] * hn[i];
            }
            y = quad_sum64(y);
        }
        if (active && m < g.M)
            __builtin_nontemporal_store(v4i{hn[0], hn[1], hn[2], hn[3]},
                                        reinterpret_cast<v4i *>(g.h + ((int64_t)m * g.D + d) * 16 + 4 * q));
        if (active && q == 0 && m < g.M) {
            const int64_t yg = ((int64_t)sat32_64(y) * s_gate[zv[t] + 128]) >> 15;
            g.yo[(int64_t)m * g.D + d] = (int8_t)clamp64(rshr64(yg, g.s_y), -127, 127);
        }
    }
}

// The batched scan step with the per-channel work split over the quad
// (nstate 16, decay shift 15, x_proj as <= kTokMaxParts int32 partials per
// token; d_inner a multiple of 64).  A wave owns 64 channels c0 + [0, 64) of
// TPB tokens; a block, four waves (256 channels).  The states stream as in dt_scan_tok_kernel: load j
// of a token moves bytes [1 KB j, 1 KB (j + 1)) of the wave's 4 KB state
// tile, so lane l = 4k + q holds states 4q..4q+3 of channel c0 + 16j + k, for
// j = 0..3.  Each lane also owns one of its four channels, c0 + 16q + k, and
// runs that channel's per-channel work once: the dt_proj dot (its channel's
// KW >= R/16 words unpacked once for the TPB tokens), dm, dt, x*dt, and the
// gate of y.  The quad passes each channel's 2*dm and x*dt from its owner with
// a DPP broadcast, and the four lanes' partial sums of y = C . h meet at the
// owner in a DPP reduce-scatter.  Where dt_scan_tok_kernel's lanes each
// repeat their channel's dot, dt and gate, this kernel does that work once.
// The state update is dt_scan_tok_kernel's S24 form (update16 with the input
// term as one clamped multiply-add); y accumulates C * H and C * L in int32
// (|sum| < 2^28 over a channel's 16 states).
template <int J>
__device__ __forceinline__ int quad_bcast(int v) {
    return __builtin_amdgcn_mov_dpp(v, J * 0x55, 0xF, 0xF, false);
}
// lane q of each quad gets sum over the quad's lanes of their v[q]
__device__ __forceinline__ int quad_reduce_scatter(const int (&v)[4], int q) {
    const bool odd = q & 1;
    // exchange with lane q ^ 1: keep the two channels of this lane's parity
    int k0 = odd ? v[1] : v[0], k1 = odd ? v[3] : v[2];
    const int s0 = odd ? v[0] : v[1], s1 = odd ? v[2] : v[3];
    k0 += __builtin_amdgcn_mov_dpp(s0, 0xB1, 0xF, 0xF, false);
    k1 += __builtin_amdgcn_mov_dpp(s1, 0xB1, 0xF, 0xF, false);
    // exchange with lane q ^ 2: k0 holds channel q & 1, k1 channel (q & 1) + 2
    const bool hi = q & 2;
    const int mine = hi ? k1 : k0, other = hi ? k0 : k1;
    return mine + __builtin_amdgcn_mov_dpp(other, 0x4E, 0xF, 0xF, false);
}

template <int TPB, int KW>
__global__ __launch_bounds__(256) void dt_scan_quad_kernel(DtScanArgs g) {
    __shared__ __align__(16) int8_t s_dt[TPB][16 * KW];
    __shared__ __align__(16) int32_t s_bc[TPB][32];   // B at [0, 16), C at [16, 32), as int32
    __shared__ int32_t s_dtq[41];
    __shared__ int32_t s_gate[256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int q = lane & 3, k = lane >> 2;
    const int32_t tab_dt = kStepTables.dtq[min(tid, 40)];
    const int32_t tab_gate = kStepTables.gate[tid];
    const int m0 = blockIdx.y * TPB;
    const int c0 = blockIdx.x * 256 + (tid >> 6) * 64;
    const bool wave_on = c0 < g.D;              // uniform: the wave's 64 channels all exist
    const int cl0 = wave_on ? c0 : g.D - 64;    // loads of a wave past d_inner read the last 64 channels
    const int own = cl0 + 16 * q + k;
    const int kw = g.R / 16;   // 1 <= kw <= KW
    // every load before the first wait, the x_proj partials first (their sum
    // is staged while the states stream in).  The TPB x_proj rows: thread
    // i < TPB * nxr / 4 sums outputs 4i..4i+3 of every partial (nxr = R + 32,
    // a multiple of 16: a group never straddles two tokens or the dt_raw / B /
    // C boundaries)
    const int nxr = g.R + 32;
    const int ngrp = TPB * nxr / 4;
    const int gi = min(tid, ngrp - 1);
    const int tq = 4 * gi / nxr, cq = 4 * gi - tq * nxr;
    v4i xq4[kTokMaxParts];
    {
        const int mt = min(m0 + tq, g.M - 1);
#pragma unroll
        for (int b = 0; b < kTokMaxParts; ++b)
            xq4[b] = *reinterpret_cast<const v4i *>(g.xpart + ((int64_t)mt * g.nblk + min(b, g.nblk - 1)) * nxr + cq);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the partial loads ahead of the state loads
    // then the per-channel operands, then the wave's state tiles (token t's
    // starts at channel cl0, its load j at + 1 KB * j)
    int xsv[TPB], zv[TPB];
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        const int mt = min(m0 + t, g.M - 1);
        xsv[t] = g.xs[(int64_t)mt * g.D + own];
        zv[t] = g.z[(int64_t)mt * g.z_stride + own];
    }
    uint32_t wdt[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) wdt[i] = g.w_dt[(int64_t)own * kw + min(i, kw - 1)];  // words past kw zeroed below
    v4i b4[4];
    {
        const v4i *bp = reinterpret_cast<const v4i *>(g.base + (int64_t)(cl0 + k) * 16 + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) b4[j] = bp[64 * j];
    }
    __builtin_amdgcn_sched_barrier(0);
    v4i h[TPB][4];
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        const v4i *hp =
            reinterpret_cast<const v4i *>(g.h + ((int64_t)min(m0 + t, g.M - 1) * g.D + cl0 + k) * 16 + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) h[t][j] = __builtin_nontemporal_load(hp + 64 * j);
    }
    // words past kw are zero, so the dot runs over all KW words (dt_raw past R
    // in LDS is never written; it meets zero weights)
    v4i wt[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) wt[i] = unpack16(wdt[i] & (0u - (uint32_t)(i < kw)));  // code 0 is weight 0
    if (tid < ngrp) {
        v4i sum = xq4[0];
#pragma unroll
        for (int b = 1; b < kTokMaxParts; ++b)
            if (b < g.nblk) sum += xq4[b];
        v4i qv;
#pragma unroll
        for (int r = 0; r < 4; ++r) qv[r] = clamp32(rshr32(sum[r], g.s_x), -127, 127);
        if (cq < g.R) {
            uint32_t w = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) w |= (uint32_t)(qv[r] & 255) << (8 * r);
            *reinterpret_cast<uint32_t *>(&s_dt[tq][cq]) = w;
        } else {
            *reinterpret_cast<v4i *>(&s_bc[tq][cq - g.R]) = qv;
        }
    }
    if (tid < 41) s_dtq[tid] = tab_dt;
    s_gate[tid] = tab_gate;
    __syncthreads();
    // 2 * base, the base first clamped to [-21, 32021] (with |dm| <= 20,
    // clamp(base + dm, 0, 32000) is unchanged and the doubling cannot overflow)
    int b2[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) b2[j][e] = 2 * clamp32(b4[j][e], -21, 32021);
#pragma unroll
    for (int t = 0; t < TPB; ++t) {
        const int m = m0 + t;
        // the owned channel's dt_proj dot, dm and x * dt
        int acc = 0;
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const v4i xv = *reinterpret_cast<const v4i *>(&s_dt[t][16 * i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_sdot4(wt[i][j], xv[j], acc, false);
        }
        const int dm = clamp32(rshr32(acc, g.s_dt), -20, 20);
        // |x * dt| <= 127 * 6554: the rounded shift is exact in 32 bits
        const int xd = (__mul24(xsv[t], s_dtq[dm + 20]) + 512) >> 10;
        const int dm2 = 2 * dm;
        const int dmj[4] = {quad_bcast<0>(dm2), quad_bcast<1>(dm2), quad_bcast<2>(dm2), quad_bcast<3>(dm2)};
        const int xdj[4] = {quad_bcast<0>(xd), quad_bcast<1>(xd), quad_bcast<2>(xd), quad_bcast<3>(xd)};
        const v4i bb = *reinterpret_cast<const v4i *>(&s_bc[t][4 * q]);
        const v4i cc = *reinterpret_cast<const v4i *>(&s_bc[t][16 + 4 * q]);
        const bool store = wave_on && m < g.M;   // uniform
        v4i *hp = reinterpret_cast<v4i *>(g.h + ((int64_t)min(m, g.M - 1) * g.D + cl0 + k) * 16 + 4 * q);
        int yh[4], yl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            yh[j] = 0;
            yl[j] = 0;
            v4i hn;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int n2 = min(max(b2[j][e] + dmj[j], 0), 64000);
                int32_t hv = h[t][j][e];
                update16_b(hv, n2, bb[e], xdj[j], cc[e], yh[j], yl[j]);
                hn[e] = hv;
            }
            if (store) __builtin_nontemporal_store(hn, hp + 64 * j);
        }
        const int YH = quad_reduce_scatter(yh, q), YL = quad_reduce_scatter(yl, q);
        if (store) {
            const int64_t y = (int64_t)YH * 65536 + YL;
            const int64_t yg = ((int64_t)sat32_64(y) * s_gate[zv[t] + 128]) >> 15;
            g.yo[(int64_t)m * g.D + own] = (int8_t)clamp64(rshr64(yg, g.s_y), -127, 127);
        }
    }
}

template <int TPB>
void launch_scan_quad(int kw, dim3 grid, hipStream_t hs, const DtScanArgs &g) {
    if (kw <= 4) hipLaunchKernelGGL((dt_scan_quad_kernel<TPB, 4>), grid, dim3(256), 0, hs, g);
    else if (kw <= 8) hipLaunchKernelGGL((dt_scan_quad_kernel<TPB, 8>), grid, dim3(256), 0, hs, g);
    else hipLaunchKernelGGL((dt_scan_quad_kernel<TPB, 16>), grid, dim3(256), 0, hs, g);
}

template <int NPL>
void launch_xproj_scan(int ntiles, dim3 grid, hipStream_t hs, const DtScanArgs &g) {
    if (ntiles <= 2) hipLaunchKernelGGL((dt_scan_step_kernel<2, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles == 3) hipLaunchKernelGGL((dt_scan_step_kernel<3, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles == 4) hipLaunchKernelGGL((dt_scan_step_kernel<4, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles == 5) hipLaunchKernelGGL((dt_scan_step_kernel<5, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles == 6) hipLaunchKernelGGL((dt_scan_step_kernel<6, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles <= 8) hipLaunchKernelGGL((dt_scan_step_kernel<8, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles <= 10) hipLaunchKernelGGL((dt_scan_step_kernel<10, NPL>), grid, dim3(256), 0, hs, g);
    else if (ntiles <= 12) hipLaunchKernelGGL((dt_scan_step_kernel<12, NPL>), grid, dim3(256), 0, hs, g);
    else hipLaunchKernelGGL((dt_scan_step_kernel<16, NPL>), grid, dim3(256), 0, hs, g);
}

mi_status check_norm_gemv(const char *fn, const int32_t *r, const int64_t *row_stats, int stats_parts,
                          const int16_t *gamma, const uint8_t *w, int m, int n, int k) {
    MI_REQUIRE(m >= 0 && n >= 0 && k >= 0, MI_ERR_BAD_DIM, "%s: negative size", fn);
    MI_REQUIRE(m <= kMaxRows * kMaxRowGroups, MI_ERR_BAD_DIM, "%s: m=%d exceeds %d tokens", fn, m,
               kMaxRows * kMaxRowGroups);
    MI_REQUIRE(k % 64 == 0 && k <= kMaxNormK, MI_ERR_BAD_DIM, "%s: k=%d must be a multiple of 64 and <= %d", fn, k,
               kMaxNormK);
    if ((int64_t)m * n == 0) return MI_OK;
    MI_REQUIRE(r && gamma && w, MI_ERR_NULL_POINTER, "%s: r, gamma and w_packed are required", fn);
    MI_REQUIRE(aligned(w, 16) && aligned(gamma, 8), MI_ERR_BAD_ALIGNMENT,
               "%s: w_packed must be 16-byte aligned, gamma 8-byte aligned", fn);
    if (row_stats) {
        MI_REQUIRE(stats_parts >= 1 && stats_parts <= kMaxStatParts, MI_ERR_BAD_ARG,
                   "%s: stats_parts=%d outside [1,%d]", fn, stats_parts, kMaxStatParts);
        MI_REQUIRE(aligned(row_stats, stats_parts > 1 ? 16 : 8), MI_ERR_BAD_ALIGNMENT,
                   "%s: row_stats must be 8-byte aligned (16-byte with stats_parts > 1)", fn);
    }
    return MI_OK;
}

size_t norm_gemv_lds(int k) { return (size_t)kMaxRows * (k + 16) + 4 * 64 * sizeof(v4i); }

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status mi_norm_bitlinear(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                       const int16_t *gamma, const uint8_t *w_packed, void *out, int ldo, int kind,
                                       int m, int n, int k, int shift, void *stream) {
    clear_error();
    mi_status st = check_norm_gemv("mi_norm_bitlinear", r, row_stats, stats_parts, gamma, w_packed, m, n, k);
    if (st != MI_OK || (int64_t)m * n == 0) return st;
    MI_REQUIRE(kind == MI_OUT_INT8 || kind == MI_OUT_INT32, MI_ERR_BAD_ARG,
               "mi_norm_bitlinear: kind %d (INT8 or INT32 only)", kind);
    MI_REQUIRE(out && ldo >= n, MI_ERR_BAD_DIM, "mi_norm_bitlinear: out required with ldo >= n");
    MI_REQUIRE(shift >= 0 && shift <= 30, MI_ERR_BAD_ARG, "mi_norm_bitlinear: shift=%d outside [0,30]", shift);
    NormGemvArgs g{};
    MI_REQUIRE(aligned(r, 16), MI_ERR_BAD_ALIGNMENT, "mi_norm_bitlinear: r must be 16-byte aligned");
    g.r = r; g.row_stats = row_stats; g.stats_parts = stats_parts; g.gamma = gamma;
    g.w = reinterpret_cast<const uint32_t *>(w_packed); g.out = out; g.ldo = ldo;
    g.M = m; g.N = n; g.K = k; g.kw = k / 16; g.shift = shift;
    // wide blocks (64 features) once there are enough of them to fill the GPU
    const bool wide = n >= 16384;
    const dim3 grid((unsigned)(wide ? (n + 63) / 64 : (n + 15) / 16), (unsigned)((m + kMaxRows - 1) / kMaxRows));
    const size_t lds = norm_gemv_lds(k);
    hipStream_t hs = as_stream(stream);
    if (kind == MI_OUT_INT32) {
        if (wide) hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT32, false, true>), grid, dim3(256), lds, hs, g);
        else hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT32, false, false>), grid, dim3(256), lds, hs, g);
    } else {
        if (wide) hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT8, false, true>), grid, dim3(256), lds, hs, g);
        else hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT8, false, false>), grid, dim3(256), lds, hs, g);
    }
    return check_launch("mi_norm_bitlinear");
}

extern "C" mi_status mi_norm_bitlinear_argmax(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                              const int16_t *gamma, const uint8_t *w_packed, int32_t *logits, int ldo,
                                              int64_t *keys, int m, int n, int k, void *stream) {
    clear_error();
    mi_status st =
        check_norm_gemv("mi_norm_bitlinear_argmax", r, row_stats, stats_parts, gamma, w_packed, m, n, k);
    if (st != MI_OK || (int64_t)m * n == 0) return st;
    MI_REQUIRE(keys, MI_ERR_NULL_POINTER, "mi_norm_bitlinear_argmax: keys is required");
    MI_REQUIRE(!logits || ldo >= n, MI_ERR_BAD_DIM, "mi_norm_bitlinear_argmax: ldo=%d < n=%d", ldo, n);
    MI_REQUIRE(aligned(r, 16), MI_ERR_BAD_ALIGNMENT, "mi_norm_bitlinear_argmax: r must be 16-byte aligned");
    NormGemvArgs g{};
    g.r = r; g.row_stats = row_stats; g.stats_parts = stats_parts; g.gamma = gamma;
    g.w = reinterpret_cast<const uint32_t *>(w_packed); g.out = logits; g.ldo = ldo; g.keys = keys;
    g.M = m; g.N = n; g.K = k; g.kw = k / 16; g.shift = 0;
    hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT32, false, true>),
                       dim3((unsigned)((n + 63) / 64), (unsigned)((m + kMaxRows - 1) / kMaxRows)), dim3(256),
                       norm_gemv_lds(k), as_stream(stream), g);
    return check_launch("mi_norm_bitlinear_argmax");
}

namespace mi {
namespace {
mi_status norm_in_proj_conv_impl(const char *fn, bool norm_v2, const int32_t *r, const int64_t *row_stats,
                                 int stats_parts, const int16_t *gamma, const uint8_t *w_in, int s_in, const int8_t *conv_w, const int32_t *conv_b,
                                 int8_t *conv_state, int8_t *xs, int8_t *xz, const uint8_t *w_x, int nx,
                                 int32_t *xpart, int m, int d_model, int d_inner, void *stream) {
    clear_error();
    mi_status st = check_norm_gemv(fn, r, row_stats, stats_parts, gamma, w_in, m, 2 * d_inner, d_model);
    if (st != MI_OK || (int64_t)m * d_inner == 0) return st;
    MI_REQUIRE(d_inner % 16 == 0, MI_ERR_BAD_DIM, "%s: d_inner=%d must be a multiple of 16", fn, d_inner);
    MI_REQUIRE(conv_w && conv_b && conv_state && xs && xz, MI_ERR_NULL_POINTER,
               "%s: conv_w, conv_b, conv_state, xs and xz are required", fn);
    MI_REQUIRE(aligned(conv_w, 4) && aligned(conv_state, 4) && aligned(xs, 4), MI_ERR_BAD_ALIGNMENT,
               "%s: conv_w, conv_state and xs must be 4-byte aligned", fn);
    MI_REQUIRE(s_in >= 0 && s_in <= 30, MI_ERR_BAD_ARG, "%s: s_in=%d outside [0,30]", fn, s_in);
    MI_REQUIRE(aligned(r, 16), MI_ERR_BAD_ALIGNMENT, "%s: r must be 16-byte aligned", fn);
    if (xpart) {
        MI_REQUIRE(w_x, MI_ERR_NULL_POINTER, "%s: w_x is required with xpart", fn);
        MI_REQUIRE(nx >= 1 && nx <= 16 * kMaxXTiles, MI_ERR_BAD_DIM, "%s: nx=%d outside [1,%d]", fn, nx,
                   16 * kMaxXTiles);
        MI_REQUIRE(aligned(w_x, 4) && aligned(xpart, 16), MI_ERR_BAD_ALIGNMENT,
                   "%s: w_x must be 4-byte and xpart 16-byte aligned", fn);
    }
    NormGemvArgs g{};
    g.r = r; g.row_stats = row_stats; g.stats_parts = stats_parts; g.gamma = gamma;
    g.w = reinterpret_cast<const uint32_t *>(w_in); g.out = xz;
    g.ldo = 2 * (int64_t)d_inner;
    g.M = m; g.N = 2 * d_inner; g.K = d_model; g.kw = d_model / 16; g.shift = s_in;
    g.conv_w = conv_w; g.conv_b = conv_b; g.conv_state = conv_state; g.xs = xs; g.conv_d = d_inner;
    g.w_x = reinterpret_cast<const uint32_t *>(w_x); g.nx = nx; g.xpart = xpart; g.norm_v2 = norm_v2;
    hipLaunchKernelGGL((norm_gemv_kernel<MI_OUT_INT8, true, false>),
                       dim3((unsigned)(2 * d_inner / 16), (unsigned)((m + kMaxRows - 1) / kMaxRows)), dim3(256),
                       norm_gemv_lds(d_model), as_stream(stream), g);
    return check_launch(fn);
}
}  // namespace
}  // namespace mi

extern "C" mi_status mi_norm_in_proj_conv(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                          const int16_t *gamma, const uint8_t *w_in, int s_in,
                                          const int8_t *conv_w, const int32_t *conv_b, int8_t *conv_state,
                                          int8_t *xs, int8_t *xz, int m, int d_model, int d_inner, void *stream) {
    return norm_in_proj_conv_impl("mi_norm_in_proj_conv", false, r, row_stats, stats_parts, gamma, w_in, s_in,
                                  conv_w, conv_b, conv_state, xs, xz, nullptr, 0, nullptr, m, d_model, d_inner, stream);
}

extern "C" mi_status mi_norm_v2_in_proj_conv(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                             const int16_t *gamma, const uint8_t *w_in, int s_in,
                                             const int8_t *conv_w, const int32_t *conv_b, int8_t *conv_state,
                                             int8_t *xs, int8_t *xz, int m, int d_model, int d_inner, void *stream) {
    return norm_in_proj_conv_impl("mi_norm_v2_in_proj_conv", true, r, row_stats, stats_parts, gamma, w_in, s_in,
                                  conv_w, conv_b, conv_state, xs, xz, nullptr, 0, nullptr, m, d_model, d_inner, stream);
}

extern "C" mi_status mi_norm_in_proj_conv_xpart(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                                const int16_t *gamma, const uint8_t *w_in, int s_in,
                                                const int8_t *conv_w, const int32_t *conv_b, int8_t *conv_state,
                                                int8_t *xs, int8_t *xz,
                                                const uint8_t *w_x, int nx, int32_t *xpart, int m, int d_model,
                                                int d_inner, void *stream) {
    if (!xpart) {
        mi::clear_error();
        return mi::fail(MI_ERR_NULL_POINTER, "mi_norm_in_proj_conv_xpart: xpart is required");
    }
    return norm_in_proj_conv_impl("mi_norm_in_proj_conv_xpart", false, r, row_stats, stats_parts, gamma, w_in,
                                  s_in, conv_w, conv_b, conv_state, xs, xz, w_x, nx, xpart, m, d_model, d_inner, stream);
}

extern "C" mi_status mi_dt_scan_step(const int8_t *xp, int xp_stride, int dt_rank, const uint8_t *w_dt, int s_dt,
                                     const int8_t *xs, const int8_t *z, int z_stride, int z_off, const int32_t *base,
                                     int decay_shift, int s_y, int32_t *h_state, int8_t *yo, int m, int d_inner,
                                     int nstate, void *stream) {
    clear_error();
    MI_REQUIRE(m >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_dt_scan_step: negative size");
    MI_REQUIRE(m <= 65535, MI_ERR_BAD_DIM, "mi_dt_scan_step: m=%d exceeds 65535 tokens", m);
    MI_REQUIRE(dt_rank >= 16 && dt_rank % 16 == 0 && dt_rank <= kMaxR, MI_ERR_BAD_DIM,
               "mi_dt_scan_step: dt_rank=%d must be a multiple of 16 in [16,%d]", dt_rank, kMaxR);
    MI_REQUIRE(nstate >= 1 && nstate <= kMaxN, MI_ERR_BAD_DIM, "mi_dt_scan_step: nstate=%d outside [1,%d]", nstate,
               kMaxN);
    MI_REQUIRE(dt_rank + 2 * nstate <= xp_stride, MI_ERR_BAD_DIM, "mi_dt_scan_step: xp_stride=%d too small", xp_stride);
    MI_REQUIRE(z_off >= 0 && z_off + d_inner <= z_stride, MI_ERR_BAD_DIM, "mi_dt_scan_step: z columns exceed z_stride");
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 30, MI_ERR_BAD_ARG, "mi_dt_scan_step: decay_shift outside [1,30]");
    MI_REQUIRE(s_dt >= 0 && s_dt <= 30 && s_y >= 0 && s_y <= 30, MI_ERR_BAD_ARG, "mi_dt_scan_step: shift out of range");
    if ((int64_t)m * d_inner == 0) return MI_OK;
    MI_REQUIRE(xp && w_dt && xs && z && base && h_state && yo, MI_ERR_NULL_POINTER,
               "mi_dt_scan_step: a required pointer is NULL");
    MI_REQUIRE(aligned(w_dt, 4), MI_ERR_BAD_ALIGNMENT, "mi_dt_scan_step: w_dt must be 4-byte aligned");
    DtScanArgs g{};
    g.xp = xp; g.xp_stride = xp_stride; g.R = dt_rank; g.w_dt = reinterpret_cast<const uint32_t *>(w_dt); g.s_dt = s_dt;
    g.xs = xs; g.z = z + z_off; g.z_stride = z_stride; g.base = base; g.k = decay_shift; g.s_y = s_y;
    g.h = h_state; g.yo = yo; g.M = m; g.D = d_inner; g.N = nstate;
    const dim3 grid((unsigned)((d_inner + 63) / 64), (unsigned)m);
    const bool vec = nstate == 16 && aligned(h_state, 16) && aligned(base, 16);
    // two tokens per block measured fastest at batch 64 (2.40 ms per d2048x48 step
    // against 2.44 with four, 2.54 with eight and 2.46 with one)
    if (vec && m >= 2) {
        const dim3 tgrid((unsigned)((d_inner + 63) / 64), (unsigned)((m + 1) / 2));
        if (decay_shift == 15)
            hipLaunchKernelGGL((dt_scan_tok_kernel<2, false, true>), tgrid, dim3(256), 0, as_stream(stream), g);
        else
            hipLaunchKernelGGL((dt_scan_tok_kernel<2, false, false>), tgrid, dim3(256), 0, as_stream(stream), g);
    } else if (vec) hipLaunchKernelGGL((dt_scan_step_kernel<0, 4>), grid, dim3(256), 0, as_stream(stream), g);
    else hipLaunchKernelGGL((dt_scan_step_kernel<0, 0>), grid, dim3(256), 0, as_stream(stream), g);
    return check_launch("mi_dt_scan_step");
}

extern "C" mi_status mi_xpart_dt_scan_step(const int32_t *xpart, int nblk, int s_x, int dt_rank,
                                           const uint8_t *w_dt, int s_dt, const int8_t *xs, const int8_t *z,
                                           int z_stride, int z_off, const int32_t *base, int decay_shift, int s_y,
                                           int32_t *h_state, int8_t *yo, int m, int d_inner, int nstate,
                                           void *stream) {
    clear_error();
    MI_REQUIRE(m >= 0 && d_inner >= 0 && nblk >= 1, MI_ERR_BAD_DIM, "mi_xpart_dt_scan_step: bad size");
    MI_REQUIRE(m <= 65535, MI_ERR_BAD_DIM, "mi_xpart_dt_scan_step: m=%d exceeds 65535 tokens", m);
    MI_REQUIRE(dt_rank >= 16 && dt_rank % 16 == 0 && dt_rank <= kMaxR, MI_ERR_BAD_DIM,
               "mi_xpart_dt_scan_step: dt_rank=%d must be a multiple of 16 in [16,%d]", dt_rank, kMaxR);
    MI_REQUIRE(nstate >= 1 && nstate <= kMaxN, MI_ERR_BAD_DIM, "mi_xpart_dt_scan_step: nstate=%d outside [1,%d]",
               nstate, kMaxN);
    MI_REQUIRE(dt_rank + 2 * nstate <= 16 * kMaxXTiles, MI_ERR_BAD_DIM,
               "mi_xpart_dt_scan_step: dt_rank + 2*nstate = %d exceeds %d", dt_rank + 2 * nstate, 16 * kMaxXTiles);
    MI_REQUIRE(z_off >= 0 && z_off + d_inner <= z_stride, MI_ERR_BAD_DIM,
               "mi_xpart_dt_scan_step: z columns exceed z_stride");
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 30, MI_ERR_BAD_ARG,
               "mi_xpart_dt_scan_step: decay_shift outside [1,30]");
    MI_REQUIRE(s_x >= 0 && s_x <= 30 && s_dt >= 0 && s_dt <= 30 && s_y >= 0 && s_y <= 30, MI_ERR_BAD_ARG,
               "mi_xpart_dt_scan_step: shift out of range");
    if ((int64_t)m * d_inner == 0) return MI_OK;
    MI_REQUIRE(xpart && w_dt && xs && z && base && h_state && yo, MI_ERR_NULL_POINTER,
               "mi_xpart_dt_scan_step: a required pointer is NULL");
    MI_REQUIRE(aligned(w_dt, 4), MI_ERR_BAD_ALIGNMENT, "mi_xpart_dt_scan_step: w_dt must be 4-byte aligned");
    DtScanArgs g{};
    g.xpart = xpart; g.nblk = nblk; g.s_x = s_x; g.R = dt_rank;
    g.w_dt = reinterpret_cast<const uint32_t *>(w_dt); g.s_dt = s_dt;
    g.xs = xs; g.z = z + z_off; g.z_stride = z_stride; g.base = base; g.k = decay_shift; g.s_y = s_y;
    g.h = h_state; g.yo = yo; g.M = m; g.D = d_inner; g.N = nstate;
    const dim3 grid((unsigned)((d_inner + 63) / 64), (unsigned)m);
    const bool vec = nstate == 16 && aligned(h_state, 16) && aligned(base, 16);
    const bool few = vec && nblk <= kTokMaxParts && aligned(xpart, 16);
    // the quad-split scan step where its grid still has 256 blocks (the most
    // tokens per block that does)
    const int cblk = (d_inner + 255) / 256;
    const int quad_tpb = (int64_t)cblk * ((m + 3) / 4) >= 256   ? 4
                         : (int64_t)cblk * ((m + 1) / 2) >= 256 ? 2
                         : (int64_t)cblk * m >= 256             ? 1
                                                                : 0;
    if (few && decay_shift == 15 && quad_tpb > 0 && d_inner % 64 == 0) {
        const dim3 qgrid((unsigned)cblk, (unsigned)((m + quad_tpb - 1) / quad_tpb));
        const int kw = dt_rank / 16;
        if (quad_tpb == 4) launch_scan_quad<4>(kw, qgrid, as_stream(stream), g);
        else if (quad_tpb == 2) launch_scan_quad<2>(kw, qgrid, as_stream(stream), g);
        else launch_scan_quad<1>(kw, qgrid, as_stream(stream), g);
    } else if (few && m >= 2) {
        // few partials (mi_conv_step_xpart's channel quarters): two tokens per block
        const dim3 tgrid((unsigned)((d_inner + 63) / 64), (unsigned)((m + 1) / 2));
        if (decay_shift == 15)
            hipLaunchKernelGGL((dt_scan_tok_kernel<2, true, true>), tgrid, dim3(256), 0, as_stream(stream), g);
        else
            hipLaunchKernelGGL((dt_scan_tok_kernel<2, true, false>), tgrid, dim3(256), 0, as_stream(stream), g);
    } else if (vec && decay_shift == 15)
        hipLaunchKernelGGL((dt_scan_step_kernel<-1, 4, true>), grid, dim3(256), 0, as_stream(stream), g);
    else if (vec)
        hipLaunchKernelGGL((dt_scan_step_kernel<-1, 4>), grid, dim3(256), 0, as_stream(stream), g);
    else
        hipLaunchKernelGGL((dt_scan_step_kernel<-1, 0>), grid, dim3(256), 0, as_stream(stream), g);
    return check_launch("mi_xpart_dt_scan_step");
}

extern "C" mi_status mi_xproj_dt_scan_step(const int8_t *xs, const uint8_t *w_x, int s_x, int dt_rank,
                                           const uint8_t *w_dt, int s_dt, const int8_t *z, int z_stride, int z_off,
                                           const int32_t *base, int decay_shift, int s_y, int32_t *h_state,
                                           int8_t *yo, int m, int d_inner, int nstate, void *stream) {
    clear_error();
    MI_REQUIRE(m >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_xproj_dt_scan_step: negative size");
    MI_REQUIRE(m <= 65535, MI_ERR_BAD_DIM, "mi_xproj_dt_scan_step: m=%d exceeds 65535 tokens", m);
    MI_REQUIRE(d_inner % 32 == 0, MI_ERR_BAD_DIM, "mi_xproj_dt_scan_step: d_inner=%d must be a multiple of 32",
               d_inner);
    MI_REQUIRE(dt_rank >= 16 && dt_rank % 16 == 0 && dt_rank <= kMaxR, MI_ERR_BAD_DIM,
               "mi_xproj_dt_scan_step: dt_rank=%d must be a multiple of 16 in [16,%d]", dt_rank, kMaxR);
    MI_REQUIRE(nstate >= 1 && nstate <= kMaxN, MI_ERR_BAD_DIM, "mi_xproj_dt_scan_step: nstate=%d outside [1,%d]",
               nstate, kMaxN);
    MI_REQUIRE(dt_rank + 2 * nstate <= 16 * kMaxXTiles, MI_ERR_BAD_DIM,
               "mi_xproj_dt_scan_step: dt_rank + 2*nstate = %d exceeds %d", dt_rank + 2 * nstate, 16 * kMaxXTiles);
    MI_REQUIRE(z_off >= 0 && z_off + d_inner <= z_stride, MI_ERR_BAD_DIM,
               "mi_xproj_dt_scan_step: z columns exceed z_stride");
    MI_REQUIRE(decay_shift >= 1 && decay_shift <= 30, MI_ERR_BAD_ARG, "mi_xproj_dt_scan_step: decay_shift outside [1,30]");
    MI_REQUIRE(s_x >= 0 && s_x <= 30 && s_dt >= 0 && s_dt <= 30 && s_y >= 0 && s_y <= 30, MI_ERR_BAD_ARG,
               "mi_xproj_dt_scan_step: shift out of range");
    if ((int64_t)m * d_inner == 0) return MI_OK;
    MI_REQUIRE(xs && w_x && w_dt && z && base && h_state && yo, MI_ERR_NULL_POINTER,
               "mi_xproj_dt_scan_step: a required pointer is NULL");
    MI_REQUIRE(aligned(xs, 16) && aligned(w_x, 8) && aligned(w_dt, 4), MI_ERR_BAD_ALIGNMENT,
               "mi_xproj_dt_scan_step: xs must be 16-byte aligned, w_x 8-byte and w_dt 4-byte aligned");
    DtScanArgs g{};
    g.w_x = reinterpret_cast<const uint32_t *>(w_x); g.s_x = s_x; g.R = dt_rank;
    g.x_c16 = d_inner % 256 == 0 && aligned(w_x, 16);
    g.w_dt = reinterpret_cast<const uint32_t *>(w_dt); g.s_dt = s_dt;
    g.xs = xs; g.z = z + z_off; g.z_stride = z_stride; g.base = base; g.k = decay_shift; g.s_y = s_y;
    g.h = h_state; g.yo = yo; g.M = m; g.D = d_inner; g.N = nstate;
    const dim3 grid((unsigned)((d_inner + 63) / 64), (unsigned)m);
    hipStream_t hs = as_stream(stream);
    const int ntiles = (dt_rank + 2 * nstate + 15) / 16;
    if (nstate == 16 && aligned(h_state, 16) && aligned(base, 16)) launch_xproj_scan<4>(ntiles, grid, hs, g);
    else launch_xproj_scan<0>(ntiles, grid, hs, g);
    return check_launch("mi_xproj_dt_scan_step");
}

// ------------------------------------------------ conv step + x_proj
// Decode (one token per sequence) for widths where the in_proj stage does not
// carry the conv: one block of 8 waves per token.  Each thread runs the
// depthwise conv step + squareplus of 4 channels per pass (conv1d_step.cu:
// 30-57; the state rows shift in place) and parks xs in LDS.  x_proj then runs
// on MFMA with the token as column 0 of the B operand: wave w takes the
// 256-channel slices w, w+8, ... of K for all NT 16-row tiles of the nx
// outputs, lane group q reading weight words 4q..4q+3 of a slice with one
// 16-byte load per tile, every tile's load issued before the first MFMA (rows
// past nx are clamped; their sums are never stored).  The k order inside a
// slice is permuted alike in both operands.  The waves' sums meet in LDS and
// the block writes the requantised int8 x_proj row, so the consumer
// (mi_dt_scan_step) reads nx bytes per token.
namespace mi {
namespace {

constexpr int kConvXMaxD = 8192;
constexpr int kConvXWaves = 8;

struct ConvXArgs {
    const int8_t *xz;
    int64_t xz_stride;
    const int8_t *conv_w;
    const int32_t *conv_b;
    int8_t *conv_state;   // [M][3][D]
    int8_t *xs;           // [M][D]
    const uint32_t *w_x;  // [nx][D/16] words
    int8_t *xp;           // [M][xp_stride]
    int64_t xp_stride;
    int32_t *xpart;       // [M][kConvXParts][nx] (conv_step_xpart_kernel)
    int M, D, nx, s_x;
};

template <int NT>
__global__ __launch_bounds__(64 * kConvXWaves) void conv_step_xproj_kernel(ConvXArgs g) {
    __shared__ __align__(16) int8_t s_xs[kConvXMaxD];
    __shared__ int32_t s_red[kConvXWaves][16 * NT];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_id();
    const int l16 = lane & 15, lq = lane >> 4;
    const int m = blockIdx.x;

    const int8_t *xr = g.xz + (int64_t)m * g.xz_stride;
    int8_t *st = g.conv_state + (int64_t)m * 3 * g.D;
    for (int ch = 4 * tid; ch < g.D; ch += 4 * 64 * kConvXWaves) {
        const uint32_t x = *reinterpret_cast<const uint32_t *>(xr + ch);
        const uint32_t s0 = *reinterpret_cast<const uint32_t *>(st + ch);
        const uint32_t s1 = *reinterpret_cast<const uint32_t *>(st + g.D + ch);
        const uint32_t s2 = *reinterpret_cast<const uint32_t *>(st + 2 * g.D + ch);
        const v4i cw = *reinterpret_cast<const v4i *>(g.conv_w + (int64_t)ch * 4);
        const v4i cb = *reinterpret_cast<const v4i *>(g.conv_b + ch);
        uint32_t o = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t w = (uint32_t)cw[e];
            const int32_t acc = cb[e] + (int)(int8_t)w * (int)(int8_t)(s0 >> (8 * e)) +
                                (int)(int8_t)(w >> 8) * (int)(int8_t)(s1 >> (8 * e)) +
                                (int)(int8_t)(w >> 16) * (int)(int8_t)(s2 >> (8 * e)) +
                                (int)(int8_t)(w >> 24) * (int)(int8_t)(x >> (8 * e));
            o |= (uint32_t)(sqp_q(acc) & 255) << (8 * e);
        }
        *reinterpret_cast<uint32_t *>(g.xs + (int64_t)m * g.D + ch) = o;
        *reinterpret_cast<uint32_t *>(st + ch) = s1;
        *reinterpret_cast<uint32_t *>(st + g.D + ch) = s2;
        *reinterpret_cast<uint32_t *>(st + 2 * g.D + ch) = x;
        *reinterpret_cast<uint32_t *>(&s_xs[ch]) = o;
    }
    __syncthreads();

    const int xkw = g.D / 16;
    const int nslice = g.D / 256;
    const uint32_t *wrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) wrow[t] = g.w_x + (int64_t)min(16 * t + l16, g.nx - 1) * xkw + 4 * lq;
    v4i acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
    for (int sl = wave; sl < nslice; sl += kConvXWaves) {
        v4i wv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) wv[t] = *reinterpret_cast<const v4i *>(wrow[t] + 16 * sl);
        const int w0 = 16 * sl + 4 * lq;   // this lane group's 4 words of the slice
        v4i fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            fb[j] = l16 == 0 ? *reinterpret_cast<const v4i *>(&s_xs[16 * (w0 + j)]) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t] = mfma_i8(unpack16((uint32_t)wv[t][j]), fb[j], acc[t]);
    }
    // lanes of token column 0 (l16 == 0) hold outputs 16t + 4lq + r
    if (l16 == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) *reinterpret_cast<v4i *>(&s_red[wave][16 * t + 4 * lq]) = acc[t];
    }
    __syncthreads();
    const int used = min(kConvXWaves, nslice);
    for (int n = tid; n < g.nx; n += 64 * kConvXWaves) {
        int v = 0;
        for (int w = 0; w < used; ++w) v += s_red[w][n];
        g.xp[(int64_t)m * g.xp_stride + n] = (int8_t)clamp32(rshr32(v, g.s_x), -127, 127);
    }
}

// conv_step_xpart_kernel: block (quarter q, token m) runs the conv step +
// squareplus of channels [q*D/4, (q+1)*D/4) and the exact int32 x_proj sum
// over them, so four blocks share the conv operands and x_proj weights a
// token needs (212 KB at d_inner 4096) instead of one CU pulling them all.
// 4 waves; wave w takes the quarter's 256-channel slices w, w+4, ...  The
// first conv pass's operands and the first slice's weights are loaded before
// the first wait (clamped in-bounds; unused results are not stored).
constexpr int kConvXParts = 4;
static_assert(kConvXParts <= kTokMaxParts, "the scan step sums the quarters itself");

template <int NT>
__global__ __launch_bounds__(256) void conv_step_xpart_kernel(ConvXArgs g) {
    __shared__ __align__(16) int8_t s_xs[kConvXMaxD / kConvXParts];
    __shared__ int32_t s_red[4][16 * NT];
    constexpr int kPass = 4 * 256;   // channels per conv pass of the block
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_id();
    const int l16 = lane & 15, lq = lane >> 4;
    const int part = blockIdx.x, m = blockIdx.y;
    const int C = g.D / kConvXParts;   // a multiple of 256
    const int c0 = part * C;
    const int nsl = C / 256;

    const int8_t *xr = g.xz + (int64_t)m * g.xz_stride + c0;
    int8_t *st = g.conv_state + (int64_t)m * 3 * g.D + c0;
    int8_t *xso = g.xs + (int64_t)m * g.D + c0;
    const int xkw = g.D / 16;
    const uint32_t *wrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) wrow[t] = g.w_x + (int64_t)min(16 * t + l16, g.nx - 1) * xkw + c0 / 16 + 4 * lq;
    v4i wv0[NT];
    {
        const int sl = min(wave, nsl - 1);
#pragma unroll
        for (int t = 0; t < NT; ++t) wv0[t] = *reinterpret_cast<const v4i *>(wrow[t] + 16 * sl);
    }
    struct ConvIn {
        uint32_t x, s0, s1, s2;
        v4i cw, cb;
    };
    auto conv_load = [&](int ch) {
        ConvIn c;
        c.x = *reinterpret_cast<const uint32_t *>(xr + ch);
        c.s0 = *reinterpret_cast<const uint32_t *>(st + ch);
        c.s1 = *reinterpret_cast<const uint32_t *>(st + g.D + ch);
        c.s2 = *reinterpret_cast<const uint32_t *>(st + 2 * g.D + ch);
        c.cw = *reinterpret_cast<const v4i *>(g.conv_w + (int64_t)(c0 + ch) * 4);
        c.cb = *reinterpret_cast<const v4i *>(g.conv_b + c0 + ch);
        return c;
    };
    // depthwise conv step (conv1d_step.cu:30-57) + squareplus of 4 channels
    auto conv_finish = [&](const ConvIn &c, int ch) {
        uint32_t o = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t w = (uint32_t)c.cw[e];
            const int32_t acc = c.cb[e] + (int)(int8_t)w * (int)(int8_t)(c.s0 >> (8 * e)) +
                                (int)(int8_t)(w >> 8) * (int)(int8_t)(c.s1 >> (8 * e)) +
                                (int)(int8_t)(w >> 16) * (int)(int8_t)(c.s2 >> (8 * e)) +
                                (int)(int8_t)(w >> 24) * (int)(int8_t)(c.x >> (8 * e));
            o |= (uint32_t)(sqp_q(acc) & 255) << (8 * e);
        }
        *reinterpret_cast<uint32_t *>(xso + ch) = o;
        *reinterpret_cast<uint32_t *>(st + ch) = c.s1;
        *reinterpret_cast<uint32_t *>(st + g.D + ch) = c.s2;
        *reinterpret_cast<uint32_t *>(st + 2 * g.D + ch) = c.x;
        *reinterpret_cast<uint32_t *>(&s_xs[ch]) = o;
    };
    {
        const ConvIn c = conv_load(min(4 * tid, C - 4));
        if (4 * tid < C) conv_finish(c, 4 * tid);
    }
    for (int ch = 4 * tid + kPass; ch < C; ch += kPass) conv_finish(conv_load(ch), ch);
    __syncthreads();

    v4i acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
    auto slice_mfma = [&](const v4i (&wv)[NT], int sl) {
        const int w0 = 16 * sl + 4 * lq;   // this lane group's 4 words of the slice
        v4i fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            fb[j] = l16 == 0 ? *reinterpret_cast<const v4i *>(&s_xs[16 * (w0 + j)]) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t] = mfma_i8(unpack16((uint32_t)wv[t][j]), fb[j], acc[t]);
    };
    if (wave < nsl) slice_mfma(wv0, wave);
    for (int sl = wave + 4; sl < nsl; sl += 4) {
        v4i wv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) wv[t] = *reinterpret_cast<const v4i *>(wrow[t] + 16 * sl);
        slice_mfma(wv, sl);
    }
    // lanes of token column 0 (l16 == 0) hold outputs 16t + 4lq + r
    if (l16 == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) *reinterpret_cast<v4i *>(&s_red[wave][16 * t + 4 * lq]) = acc[t];
    }
    __syncthreads();
    const int used = min(4, nsl);
    int32_t *dst = g.xpart + ((int64_t)m * kConvXParts + part) * g.nx;
    for (int n = tid; n < g.nx; n += 256) {
        int v = 0;
        for (int w = 0; w < used; ++w) v += s_red[w][n];
        dst[n] = v;
    }
}

}  // namespace
}  // namespace mi

extern "C" mi_status mi_conv_step_xpart(const int8_t *xz, int xz_stride, const int8_t *conv_w,
                                        const int32_t *conv_b, int8_t *conv_state, int8_t *xs,
                                        const uint8_t *w_x, int nx, int32_t *xpart, int m, int d_inner,
                                        void *stream) {
    using namespace mi;
    clear_error();
    MI_REQUIRE(m >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_conv_step_xpart: negative size");
    MI_REQUIRE(m <= 65535, MI_ERR_BAD_DIM, "mi_conv_step_xpart: m=%d exceeds 65535 tokens", m);
    MI_REQUIRE(d_inner % (256 * kConvXParts) == 0 && d_inner <= kConvXMaxD, MI_ERR_BAD_DIM,
               "mi_conv_step_xpart: d_inner=%d must be a multiple of %d and <= %d", d_inner, 256 * kConvXParts,
               kConvXMaxD);
    MI_REQUIRE(nx >= 1 && nx <= 16 * kMaxXTiles, MI_ERR_BAD_DIM, "mi_conv_step_xpart: nx=%d outside [1,%d]", nx,
               16 * kMaxXTiles);
    MI_REQUIRE(xz_stride >= d_inner && xz_stride % 4 == 0, MI_ERR_BAD_DIM,
               "mi_conv_step_xpart: xz_stride=%d must be >= d_inner and a multiple of 4", xz_stride);
    if ((int64_t)m * d_inner == 0) return MI_OK;
    MI_REQUIRE(xz && conv_w && conv_b && conv_state && xs && w_x && xpart, MI_ERR_NULL_POINTER,
               "mi_conv_step_xpart: a required pointer is NULL");
    MI_REQUIRE(aligned(xz, 4) && aligned(conv_w, 16) && aligned(conv_b, 16) && aligned(conv_state, 4) &&
                   aligned(xs, 4) && aligned(w_x, 16) && aligned(xpart, 4),
               MI_ERR_BAD_ALIGNMENT,
               "mi_conv_step_xpart: xz, conv_state, xs, xpart 4-byte, conv_w, conv_b, w_x 16-byte aligned");
    ConvXArgs g{};
    g.xz = xz; g.xz_stride = xz_stride; g.conv_w = conv_w; g.conv_b = conv_b; g.conv_state = conv_state; g.xs = xs;
    g.w_x = reinterpret_cast<const uint32_t *>(w_x); g.xpart = xpart;
    g.M = m; g.D = d_inner; g.nx = nx;
    const dim3 grid((unsigned)kConvXParts, (unsigned)m), block(256);
    const hipStream_t hs = as_stream(stream);
    const int nt = (nx + 15) / 16;
    if (nt <= 2) hipLaunchKernelGGL(conv_step_xpart_kernel<2>, grid, block, 0, hs, g);
    else if (nt <= 4) hipLaunchKernelGGL(conv_step_xpart_kernel<4>, grid, block, 0, hs, g);
    else if (nt <= 6) hipLaunchKernelGGL(conv_step_xpart_kernel<6>, grid, block, 0, hs, g);
    else if (nt <= 8) hipLaunchKernelGGL(conv_step_xpart_kernel<8>, grid, block, 0, hs, g);
    else if (nt <= 10) hipLaunchKernelGGL(conv_step_xpart_kernel<10>, grid, block, 0, hs, g);
    else if (nt <= 12) hipLaunchKernelGGL(conv_step_xpart_kernel<12>, grid, block, 0, hs, g);
    else hipLaunchKernelGGL(conv_step_xpart_kernel<16>, grid, block, 0, hs, g);
    return check_launch("mi_conv_step_xpart");
}

extern "C" mi_status mi_conv_step_xproj(const int8_t *xz, int xz_stride, const int8_t *conv_w,
                                        const int32_t *conv_b, int8_t *conv_state, int8_t *xs,
                                        const uint8_t *w_x, int s_x, int nx, int8_t *xp, int xp_stride, int m,
                                        int d_inner, void *stream) {
    using namespace mi;
    clear_error();
    MI_REQUIRE(m >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_conv_step_xproj: negative size");
    MI_REQUIRE(d_inner % 256 == 0 && d_inner <= kConvXMaxD, MI_ERR_BAD_DIM,
               "mi_conv_step_xproj: d_inner=%d must be a multiple of 256 and <= %d", d_inner, kConvXMaxD);
    MI_REQUIRE(nx >= 1 && nx <= 16 * kMaxXTiles, MI_ERR_BAD_DIM, "mi_conv_step_xproj: nx=%d outside [1,%d]", nx,
               16 * kMaxXTiles);
    MI_REQUIRE(xz_stride >= d_inner && xz_stride % 4 == 0 && xp_stride >= nx, MI_ERR_BAD_DIM,
               "mi_conv_step_xproj: xz_stride=%d (>= d_inner, multiple of 4) or xp_stride=%d (>= nx) too small",
               xz_stride, xp_stride);
    MI_REQUIRE(s_x >= 0 && s_x <= 30, MI_ERR_BAD_ARG, "mi_conv_step_xproj: s_x=%d outside [0,30]", s_x);
    if ((int64_t)m * d_inner == 0) return MI_OK;
    MI_REQUIRE(xz && conv_w && conv_b && conv_state && xs && w_x && xp, MI_ERR_NULL_POINTER,
               "mi_conv_step_xproj: a required pointer is NULL");
    MI_REQUIRE(aligned(xz, 4) && aligned(conv_w, 16) && aligned(conv_b, 16) && aligned(conv_state, 4) &&
                   aligned(xs, 4) && aligned(w_x, 16),
               MI_ERR_BAD_ALIGNMENT,
               "mi_conv_step_xproj: xz, conv_state, xs 4-byte, conv_w, conv_b, w_x 16-byte aligned");
    ConvXArgs g{};
    g.xz = xz; g.xz_stride = xz_stride; g.conv_w = conv_w; g.conv_b = conv_b; g.conv_state = conv_state; g.xs = xs;
    g.w_x = reinterpret_cast<const uint32_t *>(w_x); g.xp = xp; g.xp_stride = xp_stride;
    g.M = m; g.D = d_inner; g.nx = nx; g.s_x = s_x;
    const dim3 grid((unsigned)m), block(64 * kConvXWaves);
    const int nt = (nx + 15) / 16;
    if (nt <= 2) hipLaunchKernelGGL(conv_step_xproj_kernel<2>, grid, block, 0, as_stream(stream), g);
    else if (nt <= 4) hipLaunchKernelGGL(conv_step_xproj_kernel<4>, grid, block, 0, as_stream(stream), g);
    else if (nt <= 6) hipLaunchKernelGGL(conv_step_xproj_kernel<6>, grid, block, 0, as_stream(stream), g);
    else if (nt <= 8) hipLaunchKernelGGL(conv_step_xproj_kernel<8>, grid, block, 0, as_stream(stream), g);
    else if (nt <= 10) hipLaunchKernelGGL(conv_step_xproj_kernel<10>, grid, block, 0, as_stream(stream), g);
    else if (nt <= 12) hipLaunchKernelGGL(conv_step_xproj_kernel<12>, grid, block, 0, as_stream(stream), g);
    else hipLaunchKernelGGL(conv_step_xproj_kernel<16>, grid, block, 0, as_stream(stream), g);
    return check_launch("mi_conv_step_xproj");
}
