// BitLinear b1.58 on gfx950 (spec mi-spec-2, rules 2-3).
//
// acc[m,n] = sum_k a[m,k] * W[n,k], a int8, W ternary in the 2-bit word layout
// (16 weights per 32-bit word; (word >> 2j) & 0x03030303 holds 4 codes in byte
// order).  One v_perm_b32 against the byte table {0x00, 0x01, 0xFE, 0xFF}
// turns 4 codes into 4 int8 weights, so a packed word becomes one 16-byte
// MFMA operand in 4 AND/shift + 4 permute instructions.
//
// The product is computed as C^T = W * A^T with v_mfma_i32_16x16x64_i8:
// MFMA operand A = 16 weight rows (n), operand B = 16 activation rows (m).
// Lane l holds 16 consecutive k of row l%16 for k-group l/16 in both
// operands, and result register r of lane l is (n = 4*(l/16) + r, m = l%16):
// four consecutive output features of one token, i.e. one dword of int8
// output or one 16-byte vector of int32 output per lane.  (gemm32_kernel
// uses v_mfma_i32_32x32x32_i8 the same way; its layout is described there.)
//
//   prefill GEMM: 128(n) x 128(m) block tiles, 4 waves of 32 weight rows x 128
//                 tokens, K staged 128 at a time through LDS (packed weights
//                 stay packed in LDS and are unpacked in registers), double
//                 buffered, one barrier per stage (gemm_kernel); from 512 tiles
//                 up 256(n) x 128(m) tiles on 32x32x32 MFMAs with an LDS-DMA
//                 ring (gemm32_kernel).
//   decode GEMV:  m <= 64; a block owns 16 output features, its 4 waves split
//                 K; each lane streams 16-byte words of packed weights straight
//                 from HBM and unpacks them in registers.
#include "mi_mfma.hpp"

namespace mi {
namespace {

struct GemmArgs {
    const int8_t *a;
    const uint32_t *w;   // [N][K/16] words
    void *out;
    const float *x_scale;
    int64_t lda, ldo;
    int M, N, K;
    int kw;              // K / 16 words per weight row
    int shift;
    int32_t res_mult;
    int res_shift;
    int32_t res_clamp;   // RESIDUAL: |acc| bound before the residual factor (INT32_MAX: none)
    float w_scale;
    int64_t *row_stats;  // RESIDUAL: per-row (sum r, sum r^2) of the new residual, atomically added
    int64_t *stats_parts;  // RESIDUAL: [M][N/16][2] per-block (sum r, sum r^2), plain stores
};

struct RowStat {
    int64_t s1, s2;
};

// pointer types of global_load_lds (LDS-DMA) operands
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// The residual increment of one accumulator: rshr(clamp(acc, +-res_clamp) * res_mult, res_shift).
__device__ __forceinline__ int64_t residual_delta(const GemmArgs &g, int32_t acc) {
    const int32_t c = clamp32(acc, -g.res_clamp, g.res_clamp);
    return rshr64((int64_t)c * g.res_mult, g.res_shift);
}

// Epilogue for 4 consecutive features n..n+3 of token m (n % 4 == 0).  For
// RESIDUAL it returns the sum and the sum of squares of the new residual
// values it wrote (the row statistics of the next BitShiftNorm).
template <int KIND>
__device__ __forceinline__ RowStat store4(const GemmArgs &g, int m, int n, v4i acc) {
    RowStat st{0, 0};
    if (m >= g.M || n >= g.N) return st;
    const bool full = n + 3 < g.N;
    if constexpr (KIND == MI_OUT_INT8 || KIND == MI_OUT_DECAY_MOD) {
        int8_t *o = (int8_t *)g.out + (int64_t)m * g.ldo + n;
        int v[4];
        for (int r = 0; r < 4; ++r) {
            int q = rshr32(acc[r], g.shift);
            v[r] = KIND == MI_OUT_INT8 ? clamp32(q, -127, 127) : clamp32(q, -20, 20);
        }
        if (full) {
            *reinterpret_cast<uint32_t *>(o) = (uint32_t)(v[0] & 255) | ((uint32_t)(v[1] & 255) << 8) |
                                               ((uint32_t)(v[2] & 255) << 16) | ((uint32_t)(v[3] & 255) << 24);
        } else {
            for (int r = 0; r < 4 && n + r < g.N; ++r) o[r] = (int8_t)v[r];
        }
    } else if constexpr (KIND == MI_OUT_INT32) {
        int32_t *o = (int32_t *)g.out + (int64_t)m * g.ldo + n;
        if (full) {
            *reinterpret_cast<v4i *>(o) = acc;
        } else {
            for (int r = 0; r < 4 && n + r < g.N; ++r) o[r] = acc[r];
        }
    } else if constexpr (KIND == MI_OUT_RESIDUAL) {
        int32_t *o = (int32_t *)g.out + (int64_t)m * g.ldo + n;
        for (int r = 0; r < 4 && n + r < g.N; ++r) {
            const int64_t delta = residual_delta(g, acc[r]);
            const int32_t nv = (int32_t)clamp64((int64_t)o[r] + delta, -kResidualLimit, kResidualLimit);
            o[r] = nv;
            st.s1 += nv;
            st.s2 += (int64_t)nv * nv;
        }
    } else {  // MI_OUT_FLOAT: fp32(acc) * (w_scale * x_scale[m]) as rational_bitnet.py:208
        float *o = (float *)g.out + (int64_t)m * g.ldo + n;
        const float sc = __fmul_rn(g.w_scale, g.x_scale[m]);
        for (int r = 0; r < 4 && n + r < g.N; ++r) o[r] = __fmul_rn((float)acc[r], sc);
    }
    return st;
}

// Adds the row statistics held by the four lanes l16, l16+16, l16+32, l16+48
// (one token, sixteen features) to row_stats[m] with 64-bit atomics.
__device__ __forceinline__ void flush_row_stat(const GemmArgs &g, RowStat st, int m, int lq) {
    st.s1 += __shfl_xor(st.s1, 16);
    st.s1 += __shfl_xor(st.s1, 32);
    st.s2 += __shfl_xor(st.s2, 16);
    st.s2 += __shfl_xor(st.s2, 32);
    if (lq == 0 && m < g.M) {
        atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)m), (unsigned long long)st.s1);
        atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)m + 1), (unsigned long long)st.s2);
    }
}

// ------------------------------------------------------------ prefill GEMM
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kApitch = kBK + 16;       // bytes per staged activation row (bank-conflict free b128 reads)
constexpr int kWpitch = kBK / 16 + 4;   // words per staged weight row (conflict free b32 reads)
constexpr int kA2pitch = kBK + 32;      // activation row pitch of gemm_kernel (160 B)
// gemm_kernel's tiles per wave along n (measured at M 4096, K 768, N 3072:
// 2 -> 14.6 us, 4 -> 15.5 us, 8 -> 20.7 us; pitch 144 B instead of 160 B:
// 15.6 us)
constexpr int kGemmNI = 2;
constexpr int kGroupM = 8;            // m-tiles per group of the GEMM tile order
constexpr int kOpitch = 144;            // int8 output tile pitch in LDS (conflict-free dword writes)

// gemm_kernel: 128(n) x 128(m) block tile, 4 waves stacked along n (each 32
// weight rows x all 128 tokens, so every unpacked weight fragment feeds 8
// MFMAs), K staged 128 at a time, double buffered, one barrier per stage.
// Loads are branch-free: token and weight rows are clamped to the last valid
// row (their products only reach outputs that are never stored) and the
// weight words of a K tail beyond k are zeroed when staged.  Each thread
// fetches 4 x 16 activation bytes and one 16-byte run of 4 weight words per
// stage.  158 VGPRs: three blocks per CU (the waves-per-EU hint of 2 leaves the
// scheduler room and measured faster than 3 at the same occupancy).
//
// LDSOUT (int8 and decay-mod outputs with 16-byte aligned rows): the
// requantised tile goes through LDS and leaves as whole 128-byte row segments
// in 16-byte stores, instead of one dword per lane.
struct GemmStage {
    v4i a0, a1, a2, a3;
    v4i w;
    int wmask;   // 0 for the weight words of a K tail beyond k
};

// The in_proj GEMM of a prefill with the depthwise conv + squareplus of the x
// half in its epilogue (gemm_conv_kernel).  Blocks [0, x_blocks) own x-half
// tiles whose 128 staged token rows start 3 rows before the 125 rows they
// store, so the conv window of every stored row lies in the block's own tile;
// the other blocks own plain 128-row z-half tiles.
constexpr int kConvRows = kBM - 3;
struct ConvArgs {
    const int8_t *w;        // [D][4] taps, w[c][j] multiplies x[t - 3 + j]
    const int32_t *b;       // [D]
    const int8_t *st_in;    // [batch][3][D] x[-3..-1] per sequence, or null (zeros)
    int8_t *st_out;         // [batch][3][D] the last three x rows of each sequence
    int8_t *xs;             // [M][D] squareplus(conv(x))
    int D, L;               // d_inner, tokens per sequence (M = batch * L)
    int x_blocks;           // ceil(M / kConvRows) * D / kBN
};

// Tile t of an mtiles x ntiles grid in groups of kGroupM m-tiles: within a
// group the m-tile runs fastest and the n-tiles sweep (a bijection on
// [0, mtiles * ntiles); the last group may hold fewer m-tiles).
__device__ __forceinline__ void grouped_tile(int t, int mtiles, int ntiles, int &mt, int &nt) {
    const int per_group = kGroupM * ntiles;
    const int first_m = (t / per_group) * kGroupM;
    const int gsize = min(mtiles - first_m, kGroupM);
    const int r = t % per_group;
    mt = first_m + r % gsize;
    nt = r / gsize;
}

template <int KIND, bool LDSOUT, int NI, bool CONV>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, const ConvArgs &cv) {
    // each wave computes NI x MJ tiles of 16 x 16 outputs: NI along n (weight
    // rows), MJ along m (tokens); the four waves tile the 128 x 128 block as
    // WN x WM
    constexpr int MJ = 16 / NI;
    constexpr int WN = 8 / NI, WM = 4 / WN;
    static_assert(NI * MJ == 16 && WN * WM == 4 && WN * NI == 8 && WM * MJ == 8, "wave tiling");
    __shared__ __align__(16) int8_t sA[2][kBM * kA2pitch];
    __shared__ __align__(16) uint32_t sW[2][kBN * kWpitch];
    static_assert(kBM * kOpitch <= kBM * kA2pitch, "output tile must fit one activation buffer");
    static_assert(kBK == 128, "the stage loop below is written for two 64-deep halves");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = wave_id();
    const int wn = wid / WM, wm = wid % WM;
    const int l16 = lane & 15, lq = lane >> 4;

    // Tile order: the dispatcher deals consecutive block ids to the 8 XCDs in
    // turn, so block b works on tile id (b % 8) * (T / 8) + b / 8 and each XCD
    // owns a contiguous run of ids; along that run the tiles go in groups of
    // kGroupM m-tiles with the n-tiles sweeping within a group (grouped_tile).
    // The ~96 tiles an XCD runs at once then share 8 activation m-tiles and
    // about 12 weight n-tiles in its L2; with m-fastest ids an XCD's concurrent
    // tiles touched 32 m-tiles, more activation rows than one L2 holds at
    // large M (32768 x 2048 -> 8192: 633 -> 554 us).  The conv form orders its
    // x-half tiles and its z-half tiles each this way.
    int m0, n0;
    bool xblk = false;   // block-uniform: a conv x-half tile
    {
        // a contiguous run of ids per XCD within [0, T) (the conv form: within
        // the x-half and the z-half tiles separately, so every XCD gets its
        // share of the heavier x-half epilogues)
        auto xcd_run = [](int b, int T) { return (T & 7) == 0 ? (b & 7) * (T >> 3) + (b >> 3) : b; };
        int t = (int)blockIdx.x;
        if constexpr (CONV) {
            const int zb = (int)gridDim.x - cv.x_blocks;
            t = (cv.x_blocks & 7) == 0 ? (t < cv.x_blocks ? xcd_run(t, cv.x_blocks) : cv.x_blocks + xcd_run(t - cv.x_blocks, zb))
                                       : t;
        } else {
            t = xcd_run(t, (int)gridDim.x);
        }
        if constexpr (CONV) {
            if (t < cv.x_blocks) {
                const int xmt = (g.M + kConvRows - 1) / kConvRows;
                xblk = true;
                int mt, nt;
                grouped_tile(t, xmt, cv.D / kBN, mt, nt);
                m0 = mt * kConvRows - 3;
                n0 = nt * kBN;
            } else {
                const int mtiles = (g.M + kBM - 1) / kBM;
                int mt, nt;
                grouped_tile(t - cv.x_blocks, mtiles, (g.N - cv.D + kBN - 1) / kBN, mt, nt);
                m0 = mt * kBM;
                n0 = cv.D + nt * kBN;
            }
        } else {
            int mt, nt;
            grouped_tile(t, (g.M + kBM - 1) / kBM, (g.N + kBN - 1) / kBN, mt, nt);
            m0 = mt * kBM;
            n0 = nt * kBN;
        }
    }
    const int nk = (g.K + kBK - 1) / kBK;

    const int arow = tid >> 3, ac16 = tid & 7;   // activation rows arow + 32j, 16 bytes at k = 16 * ac16
    const int wrow = tid >> 1, wh = tid & 1;     // weight row wrow, words 4 * wh .. 4 * wh + 3
    const int8_t *pa[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // rows before the first (the halo of the first x-half tile) read row 0;
        // rows past the last read row M - 1: neither reaches a stored output
        int m = min(m0 + arow + 32 * j, g.M - 1);
        if constexpr (CONV) m = max(m, 0);
        pa[j] = g.a + (int64_t)m * g.lda + ac16 * 16;
    }
    const uint32_t *pw = g.w + (int64_t)min(n0 + wrow, g.N - 1) * g.kw + wh * 4;

    GemmStage S;
    auto load = [&](int kt) {
        const int off = kt * kBK + ac16 * 16 < g.K ? kt * kBK : 0;
        S.a0 = *reinterpret_cast<const v4i *>(pa[0] + off);
        S.a1 = *reinterpret_cast<const v4i *>(pa[1] + off);
        S.a2 = *reinterpret_cast<const v4i *>(pa[2] + off);
        S.a3 = *reinterpret_cast<const v4i *>(pa[3] + off);
        const bool wok = kt * (kBK / 16) + wh * 4 < g.kw;
        S.w = *reinterpret_cast<const v4i *>(pw + (wok ? kt * (kBK / 16) : 0));
        S.wmask = wok ? -1 : 0;
    };
    auto store_stage = [&](int buf) {
        *reinterpret_cast<v4i *>(&sA[buf][(arow + 0) * kA2pitch + ac16 * 16]) = S.a0;
        *reinterpret_cast<v4i *>(&sA[buf][(arow + 32) * kA2pitch + ac16 * 16]) = S.a1;
        *reinterpret_cast<v4i *>(&sA[buf][(arow + 64) * kA2pitch + ac16 * 16]) = S.a2;
        *reinterpret_cast<v4i *>(&sA[buf][(arow + 96) * kA2pitch + ac16 * 16]) = S.a3;
        *reinterpret_cast<v4i *>(&sW[buf][wrow * kWpitch + wh * 4]) = S.w & S.wmask;
    };

    v4i acc[NI][MJ];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    load(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load(kt + 1);
        {
            // the two 64-deep halves of the stage: all weight words and the
            // first half's activation fragments up front; each fragment of the
            // second half is read into the register its first-half twin frees
            const uint32_t *wr = &sW[buf][(wn * NI * 16 + l16) * kWpitch + lq];
            uint32_t w0[NI], w1[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                w0[i] = wr[i * 16 * kWpitch];
                w1[i] = wr[i * 16 * kWpitch + 4];
            }
            const int8_t *ar = &sA[buf][(wm * MJ * 16 + l16) * kA2pitch + lq * 16];
            v4i fa[MJ];
#pragma unroll
            for (int j = 0; j < MJ; ++j) fa[j] = *reinterpret_cast<const v4i *>(ar + j * 16 * kA2pitch);
            v4i f[NI], h[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                f[i] = unpack16(w0[i]);
                h[i] = unpack16(w1[i]);
            }
#pragma unroll
            for (int j = 0; j < MJ; ++j) {
#pragma unroll
                for (int i = 0; i < NI; ++i) acc[i][j] = mfma_i8(f[i], fa[j], acc[i][j]);
                fa[j] = *reinterpret_cast<const v4i *>(ar + j * 16 * kA2pitch + 64);
            }
#pragma unroll
            for (int j = 0; j < MJ; ++j)
#pragma unroll
                for (int i = 0; i < NI; ++i) acc[i][j] = mfma_i8(h[i], fa[j], acc[i][j]);
        }
        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();   // after the last stage: every wave is done reading sA / sW
    }
    // output (n, m) of acc[i][j][r]: n = nb + i*16 + 4*lq + r, m = mb + j*16 + l16
    const int nb = wn * NI * 16, mb = wm * MJ * 16;

    if constexpr (LDSOUT) {
        int8_t *sO = &sA[0][0];
        // conv operands of this thread's 4 channels, loaded before the tile is requantised
        const int cg = tid & 31, ch = n0 + 4 * cg;
        uint32_t tw[4] = {0, 0, 0, 0};
        int32_t tb[4] = {0, 0, 0, 0};
        if constexpr (CONV) {
            if (xblk) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    tw[r] = *reinterpret_cast<const uint32_t *>(cv.w + (int64_t)(ch + r) * 4);
                    tb[r] = cv.b[ch + r];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < MJ; ++j)
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                uint32_t pk = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = rshr32(acc[i][j][r], g.shift);
                    const int v = KIND == MI_OUT_INT8 ? clamp32(q, -127, 127) : clamp32(q, -20, 20);
                    pk |= (uint32_t)(v & 255) << (8 * r);
                }
                *reinterpret_cast<uint32_t *>(&sO[(mb + j * 16 + l16) * kOpitch + nb + i * 16 + 4 * lq]) = pk;
            }
        __syncthreads();
        if constexpr (CONV) {
            if (xblk) {
                // depthwise conv + squareplus (spec rules 4.3-4.4) down the tile:
                // thread (cg, run) takes channels ch..ch+3 of staged rows
                // 3 + 16 run .. (16 rows; the last run 13), walking token
                // positions t of sequence sb; the window rows before a
                // sequence start come from the conv state
                const int run = tid >> 5;
                const int i0 = 3 + 16 * run, i1 = min(i0 + 16, kBM);
                int gm = m0 + i0;   // >= 0: m0 >= -3
                if (gm < g.M) {
                    int sb = gm / cv.L, t = gm - sb * cv.L;
                    auto row = [&](int i) { return *reinterpret_cast<const uint32_t *>(&sO[i * kOpitch + 4 * cg]); };
                    auto state = [&](int k) -> uint32_t {  // x[k] of sequence sb, k in [-3, -1]
                        return cv.st_in ? *reinterpret_cast<const uint32_t *>(cv.st_in + ((int64_t)sb * 3 + 3 + k) * cv.D + ch)
                                        : 0u;
                    };
                    // per-channel windows: byte j of win[r] is x[t - 3 + j] of channel
                    // ch + r once row t is shifted in (v_perm_b32 drops byte 0 and
                    // appends the new row's byte r), so the conv is one v_dot4
                    uint32_t win[4] = {0, 0, 0, 0};
                    auto push = [&](uint32_t v) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            win[r] = __builtin_amdgcn_perm(v, win[r], 0x00030201u | ((uint32_t)(4 + r) << 24));
                    };
                    // the window of the run's first row: rows of its own sequence, the
                    // conv state before the sequence start
                    for (int j = 3; j >= 1; --j) push(t - j >= 0 ? row(i0 - j) : state(t - j));
                    for (int i = i0; i < i1 && gm < g.M; ++i, ++gm) {
                        if (t == 0) {
                            if (i > i0)
                                for (int j = 3; j >= 1; --j) push(state(-j));
                            // a sequence shorter than the window keeps part of the old state
                            for (int j = 0; j < 3 - cv.L; ++j)
                                *reinterpret_cast<uint32_t *>(cv.st_out + ((int64_t)sb * 3 + j) * cv.D + ch) =
                                    state(cv.L + j - 3);
                        }
                        const uint32_t cur = row(i);
                        push(cur);
                        uint32_t o = 0;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int32_t c = __builtin_amdgcn_sdot4((int)win[r], (int)tw[r], tb[r], false);
                            o |= (uint32_t)(sqp_q(c) & 255) << (8 * r);
                        }
                        *reinterpret_cast<uint32_t *>(cv.xs + (int64_t)gm * cv.D + ch) = o;
                        if (t >= cv.L - 3)
                            *reinterpret_cast<uint32_t *>(cv.st_out + ((int64_t)sb * 3 + t - (cv.L - 3)) * cv.D + ch) = cur;
                        if (++t == cv.L) {
                            t = 0;
                            ++sb;
                        }
                    }
                }
                return;
            }
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = arow + 32 * p;
            const int gm = m0 + row, gn = n0 + ac16 * 16;
            const v4i v = *reinterpret_cast<const v4i *>(&sO[row * kOpitch + ac16 * 16]);
            if (gm < g.M && gn < g.N) {
                int8_t *o = (int8_t *)g.out + (int64_t)gm * g.ldo + gn;
                if (gn + 16 <= g.N) {
                    // streaming store: the tile is written once and not read back by this
                    // kernel (config-2 GEMM 15.2 -> 14.5 us; the config-3 prefill, whose
                    // next kernel reads the tile, unchanged at 13.94 ms)
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(o));
                } else {
                    for (int e = 0; e < 16 && gn + e < g.N; ++e) o[e] = (int8_t)(v[e >> 2] >> (8 * (e & 3)));
                }
            }
        }
    } else if constexpr (KIND == MI_OUT_RESIDUAL) {
        // residual rows read as 16-byte vectors, four token groups' loads issued
        // before any update (rows past M and groups past N read clamped in-bounds
        // addresses; their results are not stored)
        int32_t *ob = (int32_t *)g.out;
        // token groups of 4 m-tiles (or all of them) x every n-tile of the wave
        constexpr int JG = MJ < 4 ? MJ : 4;
#pragma unroll
        for (int h = 0; h < MJ / JG; ++h) {
            v4i old[JG][NI];
#pragma unroll
            for (int jj = 0; jj < JG; ++jj)
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int m = min(m0 + mb + (JG * h + jj) * 16 + l16, g.M - 1);
                    const int n = n0 + nb + i * 16 + 4 * lq;
                    old[jj][i] = *reinterpret_cast<const v4i *>(ob + (int64_t)m * g.ldo + (n < g.N ? n : 0));
                }
#pragma unroll
            for (int jj = 0; jj < JG; ++jj) {
                const int j = JG * h + jj;
                const int m = m0 + mb + j * 16 + l16;
                RowStat st{0, 0};
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int n = n0 + nb + i * 16 + 4 * lq;
                    if (m < g.M && n < g.N) {
                        v4i nv;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t delta = residual_delta(g, acc[i][j][r]);
                            nv[r] = (int32_t)clamp64((int64_t)old[jj][i][r] + delta, -kResidualLimit, kResidualLimit);
                        }
                        int32_t *o = ob + (int64_t)m * g.ldo + n;
                        if (n + 3 < g.N) {
                            *reinterpret_cast<v4i *>(o) = nv;
                        } else {
                            for (int r = 0; r < 4 && n + r < g.N; ++r) o[r] = nv[r];
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (n + r < g.N) {
                                st.s1 += nv[r];
                                st.s2 += (int64_t)nv[r] * nv[r];
                            }
                        }
                    }
                }
                if (g.row_stats) flush_row_stat(g, st, m, lq);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < MJ; ++j) {
            const int m = m0 + mb + j * 16 + l16;
#pragma unroll
            for (int i = 0; i < NI; ++i) store4<KIND>(g, m, n0 + nb + i * 16 + 4 * lq, acc[i][j]);
        }
    }
}

template <int KIND, bool LDSOUT, int NI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(GemmArgs g) {
    gemm_tile<KIND, LDSOUT, NI, false>(g, ConvArgs{});
}

// in_proj (int8 out, shifted) with the conv + squareplus of the x half fused
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_conv_kernel(GemmArgs g,
                                                                                              ConvArgs cv) {
    gemm_tile<MI_OUT_INT8, true, kGemmNI, true>(g, cv);
}

// ------------------------------------------- prefill GEMM, 256 x 128 tiles
// gemm32_kernel: the large-shape form of the prefill GEMM on
// v_mfma_i32_32x32x32_i8.  A 256(n) x 128(m) block tile, 4 waves stacked along
// n, each 64 weight rows x 128 tokens (2 x 4 accumulators of 32 x 32), so an
// activation fragment read from LDS feeds 2 MFMAs of 32x32x32 (half the LDS
// bytes per operation of the 32-row waves of gemm_kernel) and an unpacked
// weight fragment feeds 4.
//
// MFMA operands (C^T = W * A^T): lane l holds row l%32 of a 32-row fragment
// and 16 k of half h = l/32.  The k order inside a 128-deep stage is free as
// long as both operands agree: in k-step s (0..3) half h covers stage bytes
// [16q, 16q + 16) with q = 4h + s, so the 4 words of a weight row that half h
// needs in a stage are one 16-byte run (words 4h..4h+3).  Result register r of
// lane l is feature 8(r/4) + 4h + r%4 of its fragment, token l%32.
//
// Staging: every global load is a buffer_load_dwordx4 ... lds (LDS DMA, no
// VGPRs) into a ring of three stages; a wave waits only for its own loads of a
// stage (vmcnt counts them in order: 6 a stage) and a bare s_barrier then
// makes all waves' loads visible (__syncthreads would wait for every load in
// flight).  The activation tile is 128 rows x 128 bytes with 16-byte segment
// q of row r at position q ^ ((r >> 1) & 7): lane i of a DMA instruction lands
// at byte 16i, so the lane picks the segment that belongs there, and the
// fragment reads (rows l%32, one segment) fall in distinct bank groups.  Each
// wave's weight words go to its own LDS region and are read back by the lanes
// that loaded them.  The pipeline over a stage's 4 k-steps (the barrier in its
// middle, MFMAs interleaved with the next k-step's reads and unpack, loads
// three stages ahead) is described at the main loop.
//
// Requires K % 128 == 0, N % 256 == 0, 16-byte aligned a / w with lda % 16 == 0.
// Rows past M read row M - 1 (the conv x-half's halo rows before 0 read row 0)
// and their outputs are not stored.  Epilogues: int8 requant through a
// swizzled LDS tile and 16-byte row pieces; RESIDUAL read-modify-write of
// 16-byte int32 vectors with row statistics; the conv form as gemm_conv_kernel
// (x-half tiles of 128 staged rows storing the last 125).
constexpr int kG2BN = 256, kG2BM = 128, kG2BK = 128, kG2Ring = 3;
constexpr int kG2ConvRows = kG2BM - 3;
static_assert(kG2BM == kBM, "the conv grid counts z-half tiles with kBM");

struct G2Smem {
    int8_t a[kG2Ring][kG2BM * kG2BK];   // 3 x 16 KB; the int8 output tile reuses a[0..1]
    uint32_t w[kG2Ring][4][2][256];     // [stage][wave][fragment][lane * 4 + word]
};

__device__ __forceinline__ int g2_aoff(int r, int q) { return r * kG2BK + 16 * (q ^ ((r >> 1) & 7)); }
// int8 output tile [128][256]: 16-byte granule gr of row m at gr ^ (m & 15)
__device__ __forceinline__ int g2_ooff(int m, int nb) { return m * kG2BN + ((((nb >> 4) ^ (m & 15)) << 4) | (nb & 15)); }

// word 3 of a raw buffer resource (32-bit data format, no swizzle)
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ v16i mfma32_i8(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <int KIND, bool CONV>
__device__ __forceinline__ void gemm32_tile(const GemmArgs &g, const ConvArgs &cv) {
    static_assert(KIND == MI_OUT_INT8 || KIND == MI_OUT_RESIDUAL, "int8 or residual output");
    __shared__ __align__(16) G2Smem sm;
    const int tid = threadIdx.x, lane = tid & 63, wid = wave_id();
    const int l32 = lane & 31, h = lane >> 5;

    int m0, n0;
    bool xblk = false;   // block-uniform: a conv x-half tile
    {
        auto xcd_run = [](int b, int T) { return (T & 7) == 0 ? (b & 7) * (T >> 3) + (b >> 3) : b; };
        int t = (int)blockIdx.x;
        if constexpr (CONV) {
            const int zb = (int)gridDim.x - cv.x_blocks;
            t = (cv.x_blocks & 7) == 0 ? (t < cv.x_blocks ? xcd_run(t, cv.x_blocks) : cv.x_blocks + xcd_run(t - cv.x_blocks, zb))
                                       : t;
            if (t < cv.x_blocks) {
                int mt, nt;
                grouped_tile(t, (g.M + kG2ConvRows - 1) / kG2ConvRows, cv.D / kG2BN, mt, nt);
                xblk = true;
                m0 = mt * kG2ConvRows - 3;
                n0 = nt * kG2BN;
            } else {
                int mt, nt;
                grouped_tile(t - cv.x_blocks, (g.M + kG2BM - 1) / kG2BM, (g.N - cv.D) / kG2BN, mt, nt);
                m0 = mt * kG2BM;
                n0 = cv.D + nt * kG2BN;
            }
        } else {
            t = xcd_run(t, (int)gridDim.x);
            int mt, nt;
            grouped_tile(t, (g.M + kG2BM - 1) / kG2BM, g.N / kG2BN, mt, nt);
            m0 = mt * kG2BM;
            n0 = nt * kG2BN;
        }
    }
    const int nk = g.K / kG2BK;

    // DMA sources.  Activation instruction j of wave wid fills tile rows
    // 8 (4 wid + j) .. +7: lane i takes row + i / 8 and the segment that lands
    // at position i % 8.  Weight instruction f: row n0 + 64 wid + 32 f + l32,
    // words 4h .. 4h + 3 of the stage.
    // Buffer loads (buffer_load_dwordx4 ... lds), byte offsets below 2^31:
    // the compiler counts their LDS writes with vmcnt only, so the fragment
    // reads keep exact lgkmcnt waits (with the FLAT-encoded global_load_lds in
    // flight it waits for lgkmcnt(0), i.e. for the DMA).
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(g.a), 0, (int)min((int64_t)g.M * g.lda, (int64_t)INT32_MAX), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(g.w), 0, (int)min((int64_t)g.N * g.kw * 4, (int64_t)INT32_MAX), kBufferRsrcWord3);
    uint32_t aoffs[4], woffs[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 8 * (4 * wid + j) + (lane >> 3);
        const int q = (lane & 7) ^ ((r >> 1) & 7);
        int m = min(m0 + r, g.M - 1);
        if constexpr (CONV) m = max(m, 0);
        aoffs[j] = (uint32_t)((int64_t)m * g.lda + 16 * q);
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) woffs[f] = (uint32_t)(((int64_t)(n0 + 64 * wid + 32 * f + l32) * g.kw + 4 * h) * 4);
    auto issue = [&](int kt) {
        const int b = kt % kG2Ring;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t *)&sm.a[b][(4 * wid + j) * 1024], 16, aoffs[j],
                                                     (uint32_t)(kt * kG2BK), 0, 0);
#pragma unroll
        for (int f = 0; f < 2; ++f)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void_t *)&sm.w[b][wid][f][0], 16, woffs[f],
                                                     (uint32_t)(kt * (kG2BK / 4)), 0, 0);
    };

    v16i acc[2][4];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[f][j][r] = 0;

    // fragment read offsets: row l32 (+ 32 jj), segment 4h + s
    int aoff[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) aoff[s] = g2_aoff(l32, 4 * h + s);

    // Stage kt runs 4 k-steps of 8 MFMAs.  Each k-step's MFMAs are
    // interleaved (sched_group_barrier) with the fragment reads and weight
    // unpack of the next k-step, so one wave alone keeps its SIMD's MFMA pipe
    // fed.  Before step 2 every wave waits for its own loads of stage kt + 1
    // and reads its weight words of that stage during step 2 (its own region:
    // no barrier needed).  After the fragment reads of step 3 (issued in step
    // 2) the waves meet at one barrier: stage kt + 1 is then visible and stage
    // kt's buffer free, so step 3 refills that buffer with stage kt + 3 and
    // reads stage kt + 1's first fragments under its MFMAs (no LDS latency
    // exposed at a stage boundary; loads run 2.5 stages ahead).
    auto read_w = [&](int kt, v4i (&wv)[2]) {
#pragma unroll
        for (int f = 0; f < 2; ++f) wv[f] = *reinterpret_cast<const v4i *>(&sm.w[kt % kG2Ring][wid][f][lane * 4]);
    };
    auto read_frags = [&](int kt, int s, v4i (&fr)[4]) {
        const int8_t *abase = &sm.a[kt % kG2Ring][0];
#pragma unroll
        for (int j = 0; j < 4; ++j) fr[j] = *reinterpret_cast<const v4i *>(abase + j * 32 * kG2BK + aoff[s]);
    };
    auto mfmas = [&](const v4i (&u)[2], const v4i (&fr)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[0][j] = mfma32_i8(u[0], fr[j], acc[0][j]);
            acc[1][j] = mfma32_i8(u[1], fr[j], acc[1][j]);
        }
    };
    v4i fa[4], u[2], wv[2];
    issue(0);
    if (nk > 1) issue(1);
    if (nk > 2) issue(2);
    if (nk > 2)
        asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else if (nk > 1)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_w(0, wv);
    read_frags(0, 0, fa);
#pragma unroll
    for (int f = 0; f < 2; ++f) u[f] = unpack16((uint32_t)wv[f][0]);

    // DMA: refill with stage kt + 3; NEXT: a stage kt + 1 follows
    auto stage = [&](int kt, auto dma, auto next) {
        constexpr bool DMA = decltype(dma)::value, NEXT = decltype(next)::value;
        v4i wn[2];   // stage kt + 1's weight words (this wave's own loads: no barrier needed)
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            if (NEXT && s == 2) {
                if (kt + 2 < nk)
                    asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            v4i fn[4], un[2];
            read_frags(kt, s + 1, fn);
            if (NEXT && s == 2) read_w(kt + 1, wn);
#pragma unroll
            for (int f = 0; f < 2; ++f) un[f] = unpack16((uint32_t)wv[f][s + 1]);
            mfmas(u, fa);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // 1 MFMA
                if (NEXT && s == 2 && i < 2)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                   // 2 LDS reads
                else if (i < 4)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                   // 1 LDS read
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                       // 3 VALU
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) fa[j] = fn[j];
            u[0] = un[0];
            u[1] = un[1];
        }
        if constexpr (NEXT) {
            // step 3's fragments have landed; every wave's loads of stage kt + 1 too after the barrier
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            v4i fn[4], un[2];
            if constexpr (DMA) issue(kt + 3);
            read_frags(kt + 1, 0, fn);
#pragma unroll
            for (int f = 0; f < 2; ++f) un[f] = unpack16((uint32_t)wn[f][0]);
            mfmas(u, fa);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // 1 MFMA
                if (DMA && i < 6) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);     // 1 DMA load
                if (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);            // 1 LDS read
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                       // 3 VALU
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) fa[j] = fn[j];
            u[0] = un[0];
            u[1] = un[1];
            wv[0] = wn[0];
            wv[1] = wn[1];
        } else {
            mfmas(u, fa);
        }
    };
    int kt = 0;
    for (; kt + 3 < nk; ++kt) stage(kt, std::true_type{}, std::true_type{});
    for (; kt + 1 < nk; ++kt) stage(kt, std::false_type{}, std::true_type{});
    stage(kt, std::false_type{}, std::false_type{});
    // acc[f][j][4c + i]: feature n0 + 64 wid + 32 f + 8 c + 4 h + i, token m0 + 32 j + l32

    if constexpr (KIND == MI_OUT_INT8) {
        int8_t *so = &sm.a[0][0];
        const int cg = tid & 63, ch = n0 + 4 * cg;
        uint32_t tw[4] = {0, 0, 0, 0};
        int32_t tb[4] = {0, 0, 0, 0};
        if constexpr (CONV) {
            if (xblk) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    tw[r] = *reinterpret_cast<const uint32_t *>(cv.w + (int64_t)(ch + r) * 4);
                    tb[r] = cv.b[ch + r];
                }
            }
        }
        __syncthreads();   // every wave is done reading the ring (no loads are in flight)
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    uint32_t pk = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int q = rshr32(acc[f][j][4 * c + i], g.shift);
                        pk |= (uint32_t)(clamp32(q, -127, 127) & 255) << (8 * i);
                    }
                    *reinterpret_cast<uint32_t *>(&so[g2_ooff(32 * j + l32, 64 * wid + 32 * f + 8 * c + 4 * h)]) = pk;
                }
        __syncthreads();
        if constexpr (CONV) {
            if (xblk) {
                // depthwise conv + squareplus (spec rules 4.3-4.4) down the tile:
                // thread (cg, run) takes channels ch..ch+3 of staged rows
                // 3 + 32 run .. (32 rows; the last run 29), as in gemm_tile
                const int run = tid >> 6;
                const int i0 = 3 + 32 * run, i1 = min(i0 + 32, kG2BM);
                int gm = m0 + i0;
                if (gm < g.M) {
                    int sb = gm / cv.L, t = gm - sb * cv.L;
                    auto row = [&](int i) { return *reinterpret_cast<const uint32_t *>(&so[g2_ooff(i, 4 * cg)]); };
                    auto state = [&](int k) -> uint32_t {  // x[k] of sequence sb, k in [-3, -1]
                        return cv.st_in ? *reinterpret_cast<const uint32_t *>(cv.st_in + ((int64_t)sb * 3 + 3 + k) * cv.D + ch)
                                        : 0u;
                    };
                    uint32_t win[4] = {0, 0, 0, 0};
                    auto push = [&](uint32_t v) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            win[r] = __builtin_amdgcn_perm(v, win[r], 0x00030201u | ((uint32_t)(4 + r) << 24));
                    };
                    for (int j = 3; j >= 1; --j) push(t - j >= 0 ? row(i0 - j) : state(t - j));
                    for (int i = i0; i < i1 && gm < g.M; ++i, ++gm) {
                        if (t == 0) {
                            if (i > i0)
                                for (int j = 3; j >= 1; --j) push(state(-j));
                            for (int j = 0; j < 3 - cv.L; ++j)
                                *reinterpret_cast<uint32_t *>(cv.st_out + ((int64_t)sb * 3 + j) * cv.D + ch) =
                                    state(cv.L + j - 3);
                        }
                        const uint32_t cur = row(i);
                        push(cur);
                        uint32_t o = 0;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int32_t c = __builtin_amdgcn_sdot4((int)win[r], (int)tw[r], tb[r], false);
                            o |= (uint32_t)(sqp_q(c) & 255) << (8 * r);
                        }
                        *reinterpret_cast<uint32_t *>(cv.xs + (int64_t)gm * cv.D + ch) = o;
                        if (t >= cv.L - 3)
                            *reinterpret_cast<uint32_t *>(cv.st_out + ((int64_t)sb * 3 + t - (cv.L - 3)) * cv.D + ch) = cur;
                        if (++t == cv.L) {
                            t = 0;
                            ++sb;
                        }
                    }
                }
                return;
            }
        }
        // 128 rows x 16 granules: thread t stores granule t % 16 of rows t / 16 + 16 p
        const int gr = tid & 15;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int row = (tid >> 4) + 16 * p;
            const int gm = m0 + row;
            const v4i v = *reinterpret_cast<const v4i *>(&so[g2_ooff(row, 16 * gr)]);
            if (gm < g.M) __builtin_nontemporal_store(v, reinterpret_cast<v4i *>((int8_t *)g.out + (int64_t)gm * g.ldo + n0 + 16 * gr));
        }
    } else {
        int32_t *ob = (int32_t *)g.out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + 32 * j + l32;
            const int mc = min(m, g.M - 1);
            v4i old[2][4];
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    old[f][c] = *reinterpret_cast<const v4i *>(ob + (int64_t)mc * g.ldo + n0 + 64 * wid + 32 * f + 8 * c + 4 * h);
            RowStat st{0, 0};
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    v4i nv;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t delta = residual_delta(g, acc[f][j][4 * c + i]);
                        nv[i] = (int32_t)clamp64((int64_t)old[f][c][i] + delta, -kResidualLimit, kResidualLimit);
                        st.s1 += nv[i];
                        st.s2 += (int64_t)nv[i] * nv[i];
                    }
                    if (m < g.M)
                        *reinterpret_cast<v4i *>(ob + (int64_t)m * g.ldo + n0 + 64 * wid + 32 * f + 8 * c + 4 * h) = nv;
                }
            if (g.row_stats) {
                st.s1 += __shfl_xor(st.s1, 32);
                st.s2 += __shfl_xor(st.s2, 32);
                if (h == 0 && m < g.M) {
                    atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)m), (unsigned long long)st.s1);
                    atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)m + 1),
                              (unsigned long long)st.s2);
                }
            }
        }
    }
}

template <int KIND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm32_kernel(GemmArgs g) {
    gemm32_tile<KIND, false>(g, ConvArgs{});
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm32_conv_kernel(GemmArgs g,
                                                                                                ConvArgs cv) {
    gemm32_tile<MI_OUT_INT8, true>(g, cv);
}

// gemm_any_kernel: any k % 16 == 0 and 4-byte aligned weights (e.g. dt_proj
// with k = dt_rank): 4 waves of 64x64, weights fetched one word per thread.
// 64-deep halves of a stage that lie wholly past K are skipped (k = 48 has
// one).  LDSOUT: int8 tiles leave through LDS as whole 16-byte row pieces
// (requires ldo % 16 == 0 and a 16-byte aligned output), as in gemm_tile.
template <int KIND, bool LDSOUT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void gemm_any_kernel(GemmArgs g) {
    __shared__ __align__(16) int8_t sA[2][kBM * kApitch];
    __shared__ __align__(16) uint32_t sW[2][kBN * kWpitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_id();
    const int wn = wave >> 1, wm = wave & 1;
    const int l16 = lane & 15, lq = lane >> 4;

    const int mtiles = (g.M + kBM - 1) / kBM;
    const int m0 = (blockIdx.x % mtiles) * kBM;
    const int n0 = (blockIdx.x / mtiles) * kBN;

    uint4 ra[4];
    uint32_t rw[4];
    auto load_stage = [&](int k0) {
        for (int j = 0; j < 4; ++j) {
            const int i = tid + 256 * j;         // 1024 pieces of 16 bytes
            const int row = i >> 3, c16 = i & 7;
            const int m = m0 + row, k = k0 + c16 * 16;
            ra[j] = (m < g.M && k < g.K) ? *reinterpret_cast<const uint4 *>(g.a + (int64_t)m * g.lda + k)
                                         : make_uint4(0, 0, 0, 0);
        }
        for (int j = 0; j < 4; ++j) {
            const int i = tid + 256 * j;         // 1024 words
            const int row = i >> 3, c = i & 7;
            const int n = n0 + row, kw = (k0 >> 4) + c;
            rw[j] = (n < g.N && kw < g.kw) ? g.w[(int64_t)n * g.kw + kw] : 0u;
        }
    };
    auto store_stage = [&](int buf) {
        for (int j = 0; j < 4; ++j) {
            const int i = tid + 256 * j;
            const int row = i >> 3, c16 = i & 7;
            *reinterpret_cast<uint4 *>(&sA[buf][row * kApitch + c16 * 16]) = ra[j];
        }
        for (int j = 0; j < 4; ++j) {
            const int i = tid + 256 * j;
            const int row = i >> 3, c = i & 7;
            sW[buf][row * kWpitch + c] = rw[j];
        }
    };

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int nk = (g.K + kBK - 1) / kBK;
    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage((kt + 1) * kBK);
        for (int ks = 0; ks < kBK / 64; ++ks) {
            if (kt * kBK + ks * 64 >= g.K) break;  // block-uniform: the rest of the stage is zero padding
            v4i fw[4], fa[4];
            for (int i = 0; i < 4; ++i) {
                const int row = wn * 64 + i * 16 + l16;
                fw[i] = unpack16(sW[buf][row * kWpitch + ks * 4 + lq]);
            }
            for (int j = 0; j < 4; ++j) {
                const int row = wm * 64 + j * 16 + l16;
                fa[j] = *reinterpret_cast<const v4i *>(&sA[buf][row * kApitch + ks * 64 + lq * 16]);
            }
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_i8(fw[i], fa[j], acc[i][j]);
        }
        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

    if constexpr (LDSOUT) {
        // the requantised tile as dwords into LDS (the loop's last barrier
        // freed the staging buffers), then 16-byte pieces of whole rows out
        static_assert(KIND == MI_OUT_INT8 || KIND == MI_OUT_DECAY_MOD, "int8 tiles only");
        int8_t *sO = &sA[0][0];
        static_assert(kBM * kOpitch <= 2 * kBM * kApitch, "output tile must fit the staging buffers");
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t pk = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = rshr32(acc[i][j][r], g.shift);
                    const int v = KIND == MI_OUT_INT8 ? clamp32(q, -127, 127) : clamp32(q, -20, 20);
                    pk |= (uint32_t)(v & 255) << (8 * r);
                }
                *reinterpret_cast<uint32_t *>(&sO[(wm * 64 + j * 16 + l16) * kOpitch + wn * 64 + i * 16 + 4 * lq]) = pk;
            }
        __syncthreads();
        const int arow = tid >> 3, ac16 = tid & 7;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = arow + 32 * p;
            const int gm = m0 + row, gn = n0 + ac16 * 16;
            if (gm < g.M && gn < g.N) {
                const v4i v = *reinterpret_cast<const v4i *>(&sO[row * kOpitch + ac16 * 16]);
                int8_t *o = (int8_t *)g.out + (int64_t)gm * g.ldo + gn;
                if (gn + 16 <= g.N) {
                    __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(o));
                } else {
                    for (int e = 0; e < 16 && gn + e < g.N; ++e) o[e] = (int8_t)(v[e >> 2] >> (8 * (e & 3)));
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm * 64 + j * 16 + l16;
        RowStat st{0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const RowStat e = store4<KIND>(g, m, n0 + wn * 64 + i * 16 + 4 * lq, acc[i][j]);
            st.s1 += e.s1;
            st.s2 += e.s2;
        }
        if (KIND == MI_OUT_RESIDUAL && g.row_stats) flush_row_stat(g, st, m, lq);
    }
}

// -------------------------------------------------------------- decode GEMV
// Block = 4 waves owning 16 output features; wave w takes the 256-wide K
// super-steps w, w+4, ...  Lane (r = l%16, q = l/16) loads words
// [16s + 4q, 16s + 4q + 4) of weight row n0 + r (one 16-byte load when the
// row pitch allows it) and feeds MFMA j with word 16s + 4q + j against
// activation bytes k = 16*(16s + 4q + j) .. +16 of token 16t + r.
template <int MT, int KIND, bool VEC>
__global__ __launch_bounds__(256) void gemv_kernel(GemmArgs g) {
    __shared__ v4i red[3][MT][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = wave_id();
    const int l16 = lane & 15, lq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int n = n0 + l16;
    const int nsuper = (g.kw + 15) / 16;

    auto load_w = [&](int s, uint32_t *wv) {
        const int w0 = 16 * s + 4 * lq;
        if (VEC) {
            if (s < nsuper && n < g.N && w0 < g.kw) {
                const uint4 q = *reinterpret_cast<const uint4 *>(g.w + (int64_t)n * g.kw + w0);
                wv[0] = q.x; wv[1] = q.y; wv[2] = q.z; wv[3] = q.w;
            } else {
                wv[0] = wv[1] = wv[2] = wv[3] = 0u;
            }
        } else {
            for (int j = 0; j < 4; ++j)
                wv[j] = (s < nsuper && n < g.N && w0 + j < g.kw) ? g.w[(int64_t)n * g.kw + w0 + j] : 0u;
        }
    };

    // the residual values wave 0 will update, fetched before the product
    int32_t rpre[MT][4];
    if (KIND == MI_OUT_RESIDUAL && wave == 0) {
        for (int t = 0; t < MT; ++t) {
            const int m = 16 * t + l16, nf = n0 + 4 * lq;
            for (int r = 0; r < 4; ++r)
                rpre[t][r] = (m < g.M && nf + r < g.N) ? ((const int32_t *)g.out)[(int64_t)m * g.ldo + nf + r] : 0;
        }
    }

    v4i acc[MT];
    for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};
    uint32_t cur[4], nxt[4];
    load_w(wave, cur);
    for (int s = wave; s < nsuper; s += 4) {
        load_w(s + 4, nxt);  // next super-step's words in flight during this one
        const int w0 = 16 * s + 4 * lq;
        for (int j = 0; j < 4; ++j) {
            const v4i fw = unpack16(cur[j]);
            const int k = 16 * (w0 + j);
            for (int t = 0; t < MT; ++t) {
                const int m = 16 * t + l16;
                v4i fa = v4i{0, 0, 0, 0};
                if (m < g.M && k < g.K) fa = *reinterpret_cast<const v4i *>(g.a + (int64_t)m * g.lda + k);
                acc[t] = mfma_i8(fw, fa, acc[t]);
            }
        }
        for (int j = 0; j < 4; ++j) cur[j] = nxt[j];
    }
    if (wave > 0)
        for (int t = 0; t < MT; ++t) red[wave - 1][t][lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
        for (int t = 0; t < MT; ++t) {
            v4i v = acc[t] + red[0][t][lane] + red[1][t][lane] + red[2][t][lane];
            const int m = 16 * t + l16, nf = n0 + 4 * lq;
            if constexpr (KIND == MI_OUT_RESIDUAL) {
                // RESIDUAL from the prefetched values (same rule as store4)
                RowStat st{0, 0};
                if (m < g.M && nf < g.N) {
                    int32_t *o = (int32_t *)g.out + (int64_t)m * g.ldo + nf;
                    for (int r = 0; r < 4 && nf + r < g.N; ++r) {
                        const int64_t delta = residual_delta(g, v[r]);
                        const int32_t nv = (int32_t)clamp64((int64_t)rpre[t][r] + delta, -kResidualLimit,
                                                            kResidualLimit);
                        o[r] = nv;
                        st.s1 += nv;
                        st.s2 += (int64_t)nv * nv;
                    }
                }
                if (g.row_stats) flush_row_stat(g, st, m, lq);
            } else {
                store4<KIND>(g, m, nf, v);
            }
        }
    }
}

// --------------------------------------- batched decode GEMV, 16 < m <= 64
// One step of up to 64 sequences: every block owns FT x 16 output features
// and all four 16-token tiles; its WAVES waves take 16-word chunks of K (c,
// c + WAVES, ...), two chunks in flight (one with 16 waves).  In a chunk, lane (row l16, group
// lq) reads words [16c+4lq, 16c+4lq+4) of each of its FT weight rows with one
// 16-byte load and the 64 activation bytes of the same k of each token tile;
// all loads are unconditional from clamped addresses (a clamped row or token
// only feeds results that are not stored; a chunk past the end is re-read and
// its products skipped).  The waves' partial sums meet in LDS: up to 8 waves
// store them as 16-byte vectors (WAVES x FT x 4 x 1 KB) and waves 0-3 add
// them up for one token tile each; 16 waves add into one copy with integer
// atomics (exact, order-free; 2 of 3 LDS cycles were bank conflicts at
// 4 waves, where the stores measured faster).
// Requires kw % 16 == 0, 16-byte aligned w, a and lda.
template <int KIND, int FT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemv64_kernel(GemmArgs g) {
    constexpr int U = WAVES >= 16 ? 1 : 2;  // chunks in flight (16 waves: 128 VGPRs a lane)
    constexpr bool kStore = WAVES <= 8;
    __shared__ int32_t red[kStore ? 1 : FT][4][64][4];
    __shared__ v4i part[kStore ? WAVES : 1][kStore ? FT : 1][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), l16 = lane & 15, lq = lane >> 4;
    if constexpr (!kStore)
        for (int i = tid; i < FT * 4 * 64 * 4; i += 64 * WAVES) (&red[0][0][0][0])[i] = 0;
    const int n0 = blockIdx.x * 16 * FT;
    const int nchunk = g.kw / 16;
    const uint32_t *wrow[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) wrow[f] = g.w + (int64_t)min(n0 + 16 * f + l16, g.N - 1) * g.kw;
    const int8_t *arow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) arow[t] = g.a + (int64_t)min(16 * t + l16, g.M - 1) * g.lda;
    v4i acc[FT][4];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[f][t] = v4i{0, 0, 0, 0};
    for (int c0 = wave; c0 < nchunk; c0 += U * WAVES) {
        v4i wv[U][FT], xv[U][4][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + WAVES * u < nchunk ? c0 + WAVES * u : c0;
            const int w = 16 * c + 4 * lq;
#pragma unroll
            for (int f = 0; f < FT; ++f) wv[u][f] = *reinterpret_cast<const v4i *>(wrow[f] + w);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) xv[u][t][j] = *reinterpret_cast<const v4i *>(arow[t] + 16 * (w + j));
        }
        // keep every load of the chunks in flight ahead of the first product
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + WAVES * u < nchunk) {  // same for the whole wave
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int f = 0; f < FT; ++f) {
                        const v4i fw = unpack16((uint32_t)wv[u][f][j]);
#pragma unroll
                        for (int t = 0; t < 4; ++t) acc[f][t] = mfma_i8(fw, xv[u][t][j], acc[f][t]);
                    }
            }
        }
    }
    if constexpr (kStore) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
            for (int t = 0; t < 4; ++t) part[wave][f][t][lane] = acc[f][t];
    } else {
        __syncthreads();  // red zeroed
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) atomicAdd(&red[f][t][lane][r], acc[f][t][r]);
    }
    __syncthreads();
    if (wave >= 4) return;
    // wave w finishes token tile w: lane (token 16w + l16, group lq) holds
    // features n0 + 16f + 4lq + r
    const int m = 16 * wave + l16;
#pragma unroll
    for (int f = 0; f < FT; ++f) {
        v4i v;
        if constexpr (kStore) {
            v = part[0][f][wave][lane];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) v += part[w][f][wave][lane];
        } else {
            v = v4i{red[f][wave][lane][0], red[f][wave][lane][1], red[f][wave][lane][2], red[f][wave][lane][3]};
        }
        const RowStat st = store4<KIND>(g, m, n0 + 16 * f + 4 * lq, v);
        if (KIND == MI_OUT_RESIDUAL && g.row_stats) flush_row_stat(g, st, m, lq);
    }
}

// gemv64_kernel<KIND, FT, 4> with the activations staged through LDS: every
// block reads all M x K activation bytes, and read straight into MFMA operands
// (16 rows x 4 scattered 16-byte pieces per load) they cost more than the
// weights.  Here each wave copies the 64 x 256-byte activation slab of each of
// its chunks into its own LDS region with global_load_lds_dwordx4 (one load
// moves 4 whole rows x 256 bytes, no VGPRs involved), then reads the MFMA B
// operands from LDS.  Lane i of a load lands at byte 16i of its 1 KB block, so
// the lane choosing row 4r + i/16 fetches segment (i % 16) ^ (row % 16) of it:
// the XOR swizzle makes the 16 rows of an operand read fall in 16 different
// bank groups.  Same chunk ownership and results as gemv64_kernel.
constexpr int kG64Waves = 4, kG64U = 2;

// Blocks along y take 64-row groups (rows [64y, 64y + 64)): the prefill form
// for few outputs (x_proj, N <= 160, FT = 5), where 128 x 128 GEMM tiles would
// leave most CUs idle.
template <int KIND, int FT>
__global__ __launch_bounds__(64 * kG64Waves) void gemv64s_kernel(GemmArgs g) {
    constexpr int WAVES = kG64Waves, U = kG64U;
    if (gridDim.y > 1) {
        constexpr int kOutBytes = KIND == MI_OUT_INT8 || KIND == MI_OUT_DECAY_MOD ? 1 : 4;
        const int64_t m0 = 64 * (int64_t)blockIdx.y;
        g.a += m0 * g.lda;
        g.out = (char *)g.out + m0 * g.ldo * kOutBytes;
        if (g.x_scale) g.x_scale += m0;
        if (g.row_stats) g.row_stats += 2 * m0;
        g.M = min(64, g.M - (int)m0);
    }
    __shared__ __align__(16) int8_t stage[WAVES][U][64 * 256];
    static_assert(FT * 4 * 64 * 16 <= U * 64 * 256, "partial sums reuse the wave's staging region");
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), l16 = lane & 15, lq = lane >> 4;
    const int n0 = blockIdx.x * 16 * FT;
    const int nchunk = g.kw / 16;
    const uint32_t *wrow[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) wrow[f] = g.w + (int64_t)min(n0 + 16 * f + l16, g.N - 1) * g.kw;
    v4i acc[FT][4];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[f][t] = v4i{0, 0, 0, 0};
    // this lane's row and segment in each 4-row load (rows past M read row M - 1)
    const int srow = lane >> 4;
    for (int c0 = wave; c0 < nchunk; c0 += U * WAVES) {
        v4i wv[U][FT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + WAVES * u < nchunk ? c0 + WAVES * u : c0;
#pragma unroll
            for (int f = 0; f < FT; ++f) wv[u][f] = *reinterpret_cast<const v4i *>(wrow[f] + 16 * c + 4 * lq);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 4 * r + srow;
                const int seg = (lane & 15) ^ (row & 15);
                const int8_t *src = g.a + (int64_t)min(row, g.M - 1) * g.lda + 256 * c + 16 * seg;
                __builtin_amdgcn_global_load_lds((global_void_t *)src, (lds_void_t *)&stage[wave][u][r * 1024], 16, 0,
                                                 0);
            }
        }
        // the slabs are this wave's own: once its loads have landed it reads them
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + WAVES * u < nchunk) {  // same for the whole wave
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v4i xv[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        xv[t] = *reinterpret_cast<const v4i *>(
                            &stage[wave][u][(16 * t + l16) * 256 + 16 * ((4 * lq + j) ^ l16)]);
#pragma unroll
                    for (int f = 0; f < FT; ++f) {
                        const v4i fw = unpack16((uint32_t)wv[u][f][j]);
#pragma unroll
                        for (int t = 0; t < 4; ++t) acc[f][t] = mfma_i8(fw, xv[t], acc[f][t]);
                    }
                }
            }
        }
        // the next chunks' loads overwrite the slabs: every lane is done reading them
        __builtin_amdgcn_wave_barrier();
    }
    // partial sums into the wave's own region, then waves 0-3 add them up for one token tile each
    v4i *part = reinterpret_cast<v4i *>(&stage[wave][0][0]);   // [FT][4][64]
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < 4; ++t) part[(f * 4 + t) * 64 + lane] = acc[f][t];
    __syncthreads();
    const int m = 16 * wave + l16;
#pragma unroll
    for (int f = 0; f < FT; ++f) {
        v4i v = v4i{0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < WAVES; ++w)
            v += reinterpret_cast<const v4i *>(&stage[w][0][0])[(f * 4 + wave) * 64 + lane];
        const RowStat st = store4<KIND>(g, m, n0 + 16 * f + 4 * lq, v);
        if (KIND == MI_OUT_RESIDUAL && g.row_stats) flush_row_stat(g, st, m, lq);
    }
}

// ------------------------------------------- decode RESIDUAL GEMV, m <= 16
// The out_proj of one decode step (a few tokens): 16 features per block, 8
// waves taking 16-word chunks of K (c, c+8, ...).  In a chunk, lane (row
// l16, group lq) reads words [16c+4lq, 16c+4lq+4) of weight row n0+l16 in one
// 16-byte load and the 64 activation bytes of the same k of token l16, so
// every load is issued before the first MFMA and none is conditional: a
// token or feature index past the end is clamped, and its results are not
// stored; the words of a last, partial chunk past kw are read from a clamped
// address and zeroed.  The residual each output overwrites is read at kernel
// start.  Row statistics of the new residual: per-block partials with plain
// stores (stats_parts) or 64-bit atomics (row_stats).
// Requires kw % 4 == 0, 16-byte aligned w, a and lda.  Blocks along y take
// 16-token row groups (m <= 64 in one launch; the weight tile of a block is
// then shared by the row groups through L2).
// STAGE (the row groups of a batched step, m > 16): the 16 activation rows of
// each chunk go through LDS as in gemv64s_kernel (4 x global_load_lds per
// chunk, XOR-swizzled segments); segments past k are fetched from a clamped
// in-bounds offset and meet zeroed weight words.
template <bool STAGE>
__global__ __launch_bounds__(512) void resid_gemv16_kernel(GemmArgs g0) {
    GemmArgs g = g0;
    if (gridDim.y > 1) {
        const int64_t m0 = 16 * (int64_t)blockIdx.y;
        g.M = min(16, g0.M - (int)m0);
        g.a += m0 * g.lda;
        g.out = (int32_t *)g.out + m0 * g.ldo;
        if (g.stats_parts) g.stats_parts += m0 * gridDim.x * 2;
        if (g.row_stats) g.row_stats += m0 * 2;
    }
    __shared__ int32_t red[8][64][4];
    __shared__ int32_t s_new[16][17];
    __shared__ __align__(16) int8_t stage[STAGE ? 8 : 1][STAGE ? 2 : 1][STAGE ? 16 * 256 : 16];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), l16 = lane & 15, lq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int nchunk = (g.kw + 15) / 16;
    // output element of threads 0..255: token l16, feature n0 + 4lq + wave
    const int en = n0 + 4 * lq + (wave & 3);
    const bool eok = tid < 256 && l16 < g.M && en < g.N;
    int32_t *rp = (int32_t *)g.out + (int64_t)min(l16, g.M - 1) * g.ldo + min(en, g.N - 1);
    const int32_t rold = *rp;
    const uint32_t *wrow = g.w + (int64_t)min(n0 + l16, g.N - 1) * g.kw;
    const int8_t *arow = g.a + (int64_t)min(l16, g.M - 1) * g.lda;
    v4i acc = v4i{0, 0, 0, 0};
    for (int c0 = wave; c0 < nchunk; c0 += 16) {
        v4i wv[2], xv[2][4];
        bool live[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = c0 + 8 * u < nchunk ? c0 + 8 * u : c0;
            const int w = 16 * c + 4 * lq;
            const int wl = min(w, g.kw - 4);  // kw % 4 == 0: all four words in or all past the row
            live[u] = w < g.kw;
            wv[u] = *reinterpret_cast<const v4i *>(wrow + wl);
            if constexpr (STAGE) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 4 * r + (lane >> 4);
                    const int seg = (lane & 15) ^ row;
                    const int8_t *src = g.a + (int64_t)min(row, g.M - 1) * g.lda + min(256 * c + 16 * seg, g.K - 16);
                    __builtin_amdgcn_global_load_lds((global_void_t *)src, (lds_void_t *)&stage[wave][u][r * 1024],
                                                     16, 0, 0);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) xv[u][j] = *reinterpret_cast<const v4i *>(arow + 16 * (wl + j));
            }
        }
        if constexpr (STAGE) {
            // the wave's own slabs: once its loads have landed it reads them
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xv[u][j] = *reinterpret_cast<const v4i *>(&stage[wave][u][l16 * 256 + 16 * ((4 * lq + j) ^ l16)]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (c0 + 8 * u < nchunk)  // same for the whole wave
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = mfma_i8(unpack16(live[u] ? (uint32_t)wv[u][j] : 0u), xv[u][j], acc);
        if constexpr (STAGE) __builtin_amdgcn_wave_barrier();
    }
    *reinterpret_cast<v4i *>(&red[wave][lane][0]) = acc;
    __syncthreads();
    if (tid < 256) {
        const int r = wave;  // register r of the MFMA result = feature 4lq + r
        int32_t v = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) v += red[w][lane][r];
        const int64_t delta = residual_delta(g, v);
        const int32_t nv = (int32_t)clamp64((int64_t)rold + delta, -kResidualLimit, kResidualLimit);
        if (eok) *rp = nv;
        s_new[l16][4 * lq + r] = eok ? nv : 0;
    }
    if (g.row_stats || g.stats_parts) {
        __syncthreads();
        if (tid < 64) {
            // lane 4i+q sums features 4q..4q+3 of token i, then the quad adds up
            const int i = tid >> 2, q = tid & 3;
            int64_t s1 = 0, s2 = 0;
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const int64_t v = s_new[i][4 * q + f];
                s1 += v;
                s2 += v * v;
            }
            s1 = quad_sum64(s1);   // wave 0, all lanes active
            s2 = quad_sum64(s2);
            if (q == 0 && i < g.M) {
                if (g.stats_parts) {
                    *reinterpret_cast<v2l *>(g.stats_parts + 2 * ((int64_t)i * gridDim.x + blockIdx.x)) =
                        v2l{s1, s2};
                } else {
                    atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)i),
                              (unsigned long long)s1);
                    atomicAdd(reinterpret_cast<unsigned long long *>(g.row_stats + 2 * (int64_t)i + 1),
                              (unsigned long long)s2);
                }
            }
        }
    }
}

// ------------------------------------------------------------ helpers
// A call with no rows leaves each sequence's conv state as it was: the new
// state is the old one (zeros when there is none), word by word.
__global__ __launch_bounds__(256) void conv_state_carry_kernel(const uint32_t *in, uint32_t *out, int64_t words) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < words) out[i] = in ? in[i] : 0u;
}

__global__ void pack_ternary_kernel(const int8_t *w, uint32_t *p, int64_t words, int kw) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const int8_t *src = w + i * 16;  // row-major [n][k]: word i covers k = 16*(i%kw) of row i/kw
    uint32_t word = 0;
    for (int q = 0; q < 16; ++q) word |= ((uint32_t)src[q] & 3u) << (8 * (q & 3) + 2 * (q >> 2));
    p[i] = word;
}

// activation_quant_dynamic (rational_bitnet.py:102-111) in IEEE fp32, one
// block per row.
__global__ __launch_bounds__(256) void act_quant_kernel(const float *x, int8_t *xq, float *x_scale, int K) {
    __shared__ float red[256];
    const int64_t row = blockIdx.x;
    const float *xr = x + row * K;
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(xr[k]));
    red[threadIdx.x] = amax;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const float scale = fmaxf(red[0], 1e-8f);
    const float inv = __fdiv_rn(127.0f, scale);
    for (int k = threadIdx.x; k < K; k += 256) {
        float q = rintf(__fmul_rn(xr[k], inv));
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        xq[row * K + k] = (int8_t)q;
    }
    if (threadIdx.x == 0) x_scale[row] = __fdiv_rn(scale, 127.0f);
}

// ------------------------------------------------------------ dispatch
mi_status validate(const char *fn, const int8_t *a, int lda, const uint8_t *w, void *out, int ldo, int kind, int m,
                   int n, int k, int shift, int res_shift, const float *x_scale, int32_t res_clamp = 0) {
    MI_REQUIRE(m >= 0 && n >= 0 && k >= 0, MI_ERR_BAD_DIM, "%s: negative size (m=%d n=%d k=%d)", fn, m, n, k);
    MI_REQUIRE(k % 16 == 0, MI_ERR_BAD_DIM, "%s: k=%d must be a multiple of 16", fn, k);
    MI_REQUIRE(kind >= MI_OUT_INT32 && kind <= MI_OUT_FLOAT, MI_ERR_BAD_ARG, "%s: unknown output kind %d", fn, kind);
    if ((int64_t)m * n == 0) return MI_OK;
    MI_REQUIRE(a && w && out, MI_ERR_NULL_POINTER, "%s: a, w_packed and out are required", fn);
    MI_REQUIRE(lda >= k && lda % 16 == 0, MI_ERR_BAD_ALIGNMENT, "%s: lda=%d must be >= k and a multiple of 16", fn, lda);
    MI_REQUIRE(ldo >= n && ldo % 4 == 0, MI_ERR_BAD_ALIGNMENT, "%s: ldo=%d must be >= n and a multiple of 4", fn, ldo);
    MI_REQUIRE(aligned(a, 16), MI_ERR_BAD_ALIGNMENT, "%s: a must be 16-byte aligned", fn);
    MI_REQUIRE(aligned(w, 4), MI_ERR_BAD_ALIGNMENT, "%s: w_packed must be 4-byte aligned", fn);
    MI_REQUIRE(aligned(out, kind == MI_OUT_INT8 || kind == MI_OUT_DECAY_MOD ? 4 : 16), MI_ERR_BAD_ALIGNMENT,
               "%s: out is misaligned", fn);
    if (kind == MI_OUT_INT8 || kind == MI_OUT_DECAY_MOD)
        MI_REQUIRE(shift >= 0 && shift <= 30, MI_ERR_BAD_ARG, "%s: shift=%d outside [0,30]", fn, shift);
    if (kind == MI_OUT_RESIDUAL)
        MI_REQUIRE(res_shift >= 0 && res_shift <= 62, MI_ERR_BAD_ARG, "%s: res_shift=%d outside [0,62]", fn, res_shift);
    if (kind == MI_OUT_RESIDUAL)
        MI_REQUIRE(res_clamp >= 0, MI_ERR_BAD_ARG, "%s: res_clamp=%d must be >= 0 (0: no clamp)", fn, res_clamp);
    if (kind == MI_OUT_FLOAT) MI_REQUIRE(x_scale, MI_ERR_NULL_POINTER, "%s: x_scale is required for FLOAT output", fn);
    return MI_OK;
}

GemmArgs make_args(const int8_t *a, int lda, const uint8_t *w, void *out, int ldo, int m, int n, int k, int shift,
                   int32_t res_mult, int res_shift, const float *x_scale, float w_scale, int64_t *row_stats,
                   int32_t res_clamp = 0) {
    GemmArgs g{};
    g.a = a; g.w = reinterpret_cast<const uint32_t *>(w); g.out = out; g.x_scale = x_scale;
    g.lda = lda; g.ldo = ldo; g.M = m; g.N = n; g.K = k; g.kw = k / 16;
    g.shift = shift; g.res_mult = res_mult; g.res_shift = res_shift; g.w_scale = w_scale; g.row_stats = row_stats;
    g.res_clamp = res_clamp > 0 ? res_clamp : INT32_MAX;
    return g;
}

// Shapes and layouts gemm32_kernel takes: no K or N tail, 31-bit byte offsets
// for its buffer loads, and at least two of its tiles per CU (below that, e.g.
// config 2's 384 tiles of 4096 x 768 -> 3072, the 128 x 128 tiles of
// gemm_kernel are faster: 14.7 against 15.7 us).  `tiles` is the launch's
// tile count.
constexpr int64_t kG2MinTiles = 512;
bool gemm32_fits(const GemmArgs &g, int64_t tiles) {
    return g.K > 0 && g.K % kG2BK == 0 && g.N % kG2BN == 0 && g.M > 64 && aligned(g.a, 16) && g.lda % 16 == 0 &&
           aligned(g.w, 16) && (int64_t)g.M * g.lda <= INT32_MAX && (int64_t)g.N * g.kw * 4 <= INT32_MAX &&
           tiles >= kG2MinTiles;
}

template <int KIND>
hipError_t launch_gemm_kind(const GemmArgs &g, hipStream_t st) {
    const dim3 grid((unsigned)(((g.M + kBM - 1) / kBM) * ((g.N + kBN - 1) / kBN)));
    constexpr bool kInt8Out = KIND == MI_OUT_INT8 || KIND == MI_OUT_DECAY_MOD;
    if constexpr (kInt8Out || KIND == MI_OUT_INT32) {
        // few outputs (x_proj): 80 features x 64 rows per block, so each
        // 64-row activation slab is read once per 80 outputs and every CU is
        // busy (x_proj at d768, 16384 x 1536 -> 80: 12.5 -> 9.2 us; at K = 4096
        // the GEMM tiles stay faster: 43 vs 70 us)
        if (g.N <= 160 && g.M > 64 && (g.M + 63) / 64 <= 65535 && g.kw % 16 == 0 && g.kw / 16 <= 8 &&
            aligned(g.w, 16) && aligned(g.a, 16) && g.lda % 16 == 0) {
            hipLaunchKernelGGL((gemv64s_kernel<KIND, 5>), dim3((unsigned)((g.N + 79) / 80), (unsigned)((g.M + 63) / 64)),
                               dim3(256), 0, st, g);
            return hipGetLastError();
        }
    }
    if constexpr (KIND == MI_OUT_INT8 || KIND == MI_OUT_RESIDUAL) {
        const bool out_ok = KIND == MI_OUT_INT8 ? g.ldo % 16 == 0 && aligned(g.out, 16)
                                                : g.ldo % 4 == 0 && aligned(g.out, 16);
        const int64_t tiles = (int64_t)((g.M + kG2BM - 1) / kG2BM) * (g.N / kG2BN);
        if (out_ok && gemm32_fits(g, tiles)) {
            hipLaunchKernelGGL(gemm32_kernel<KIND>, dim3((unsigned)tiles), dim3(256), 0, st, g);
            return hipGetLastError();
        }
    }
    // gemm_kernel reads each weight row as 16-byte runs of 4 words
    if (g.kw % 4 != 0 || !aligned(g.w, 16)) {
        if (kInt8Out && g.ldo % 16 == 0 && aligned(g.out, 16))
            hipLaunchKernelGGL((gemm_any_kernel<KIND, kInt8Out>), grid, dim3(256), 0, st, g);
        else
            hipLaunchKernelGGL((gemm_any_kernel<KIND, false>), grid, dim3(256), 0, st, g);
        return hipGetLastError();
    }
    if (kInt8Out && g.ldo % 16 == 0 && aligned(g.out, 16))
        hipLaunchKernelGGL((gemm_kernel<KIND, kInt8Out, kGemmNI>), grid, dim3(256), 0, st, g);
    else
        hipLaunchKernelGGL((gemm_kernel<KIND, false, kGemmNI>), grid, dim3(256), 0, st, g);
    return hipGetLastError();
}

hipError_t launch_gemm(int kind, const GemmArgs &g, hipStream_t st) {
    switch (kind) {
        case MI_OUT_INT32: return launch_gemm_kind<MI_OUT_INT32>(g, st);
        case MI_OUT_INT8: return launch_gemm_kind<MI_OUT_INT8>(g, st);
        case MI_OUT_DECAY_MOD: return launch_gemm_kind<MI_OUT_DECAY_MOD>(g, st);
        case MI_OUT_RESIDUAL: return launch_gemm_kind<MI_OUT_RESIDUAL>(g, st);
        default: return launch_gemm_kind<MI_OUT_FLOAT>(g, st);
    }
}

template <int MT, int KIND>
hipError_t launch_gemv_mt(const GemmArgs &g, hipStream_t st) {
    const dim3 grid((unsigned)((g.N + 15) / 16));
    const bool vec = (g.kw % 4 == 0) && aligned(g.w, 16);
    if (vec)
        hipLaunchKernelGGL((gemv_kernel<MT, KIND, true>), grid, dim3(256), 0, st, g);
    else
        hipLaunchKernelGGL((gemv_kernel<MT, KIND, false>), grid, dim3(256), 0, st, g);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_gemv_kind(const GemmArgs &g, hipStream_t st) {
    if (KIND == MI_OUT_RESIDUAL && g.M <= 64 && g.kw % 4 == 0 && aligned(g.w, 16) && aligned(g.a, 16) &&
        g.lda % 16 == 0) {
        // 16-token row groups along y (weight tiles shared through L2)
        if (g.M > 16)
            hipLaunchKernelGGL(resid_gemv16_kernel<true>, dim3((unsigned)((g.N + 15) / 16), (unsigned)((g.M + 15) / 16)),
                               dim3(512), 0, st, g);
        else
            hipLaunchKernelGGL(resid_gemv16_kernel<false>, dim3((unsigned)((g.N + 15) / 16), 1u), dim3(512), 0, st, g);
        return hipGetLastError();
    }
    if (g.M > 16 && g.M <= 64 && g.kw % 16 == 0 && aligned(g.w, 16) && aligned(g.a, 16) && g.lda % 16 == 0) {
        // 32 features per block when that still gives >= 128 blocks; deep K
        // (many 16-word chunks per block) spreads over 8 or 16 waves
        const int nchunk = g.kw / 16;
        if ((g.N + 31) / 32 >= 128 && nchunk <= 8)
            hipLaunchKernelGGL((gemv64s_kernel<KIND, 2>), dim3((unsigned)((g.N + 31) / 32)), dim3(256), 0, st, g);
        else if (nchunk <= 8)
            hipLaunchKernelGGL((gemv64_kernel<KIND, 1, 4>), dim3((unsigned)((g.N + 15) / 16)), dim3(256), 0, st, g);
        else if (nchunk <= 16)
            hipLaunchKernelGGL((gemv64_kernel<KIND, 1, 8>), dim3((unsigned)((g.N + 15) / 16)), dim3(512), 0, st, g);
        else
            hipLaunchKernelGGL((gemv64_kernel<KIND, 1, 16>), dim3((unsigned)((g.N + 15) / 16)), dim3(1024), 0, st, g);
        return hipGetLastError();
    }
    if (g.M <= 16) return launch_gemv_mt<1, KIND>(g, st);
    if (g.M <= 32) return launch_gemv_mt<2, KIND>(g, st);
    return launch_gemv_mt<4, KIND>(g, st);
}

hipError_t launch_gemv(int kind, const GemmArgs &g, hipStream_t st) {
    switch (kind) {
        case MI_OUT_INT32: return launch_gemv_kind<MI_OUT_INT32>(g, st);
        case MI_OUT_INT8: return launch_gemv_kind<MI_OUT_INT8>(g, st);
        case MI_OUT_DECAY_MOD: return launch_gemv_kind<MI_OUT_DECAY_MOD>(g, st);
        case MI_OUT_RESIDUAL: return launch_gemv_kind<MI_OUT_RESIDUAL>(g, st);
        default: return launch_gemv_kind<MI_OUT_FLOAT>(g, st);
    }
}

enum class Path { kAuto, kGemm, kGemv };

mi_status bitlinear_impl(const char *fn, Path path, const int8_t *a, int lda, const uint8_t *w, void *out, int ldo,
                         int kind, int m, int n, int k, int shift, int32_t res_mult, int res_shift,
                         int32_t res_clamp, const float *x_scale, float w_scale, int64_t *row_stats, void *stream) {
    clear_error();
    mi_status st = validate(fn, a, lda, w, out, ldo, kind, m, n, k, shift, res_shift, x_scale, res_clamp);
    if (st != MI_OK || (int64_t)m * n == 0) return st;
    if (path == Path::kGemv) MI_REQUIRE(m <= 64, MI_ERR_BAD_DIM, "%s: the GEMV path takes m <= 64 (m=%d)", fn, m);
    if (row_stats) {
        MI_REQUIRE(kind == MI_OUT_RESIDUAL, MI_ERR_BAD_ARG, "%s: row_stats only with RESIDUAL output", fn);
        MI_REQUIRE(aligned(row_stats, 8), MI_ERR_BAD_ALIGNMENT, "%s: row_stats must be 8-byte aligned", fn);
    }
    const GemmArgs g =
        make_args(a, lda, w, out, ldo, m, n, k, shift, res_mult, res_shift, x_scale, w_scale, row_stats, res_clamp);
    const bool gemv = path == Path::kGemv || (path == Path::kAuto && m <= 64);
    hipError_t e = gemv ? launch_gemv(kind, g, as_stream(stream)) : launch_gemm(kind, g, as_stream(stream));
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status mi_bitlinear(const int8_t *a, int lda, const uint8_t *w_packed, void *out, int ldo, int kind,
                                  int m, int n, int k, int shift, int32_t res_mult, int res_shift,
                                  int32_t res_clamp, const float *x_scale, float w_scale, int64_t *row_stats,
                                  void *stream) {
    return bitlinear_impl("mi_bitlinear", Path::kAuto, a, lda, w_packed, out, ldo, kind, m, n, k, shift, res_mult,
                          res_shift, res_clamp, x_scale, w_scale, row_stats, stream);
}

extern "C" mi_status mi_bitlinear_gemm(const int8_t *a, int lda, const uint8_t *w_packed, void *out, int ldo,
                                       int kind, int m, int n, int k, int shift, int32_t res_mult, int res_shift,
                                       int32_t res_clamp, const float *x_scale, float w_scale, int64_t *row_stats,
                                       void *stream) {
    return bitlinear_impl("mi_bitlinear_gemm", Path::kGemm, a, lda, w_packed, out, ldo, kind, m, n, k, shift,
                          res_mult, res_shift, res_clamp, x_scale, w_scale, row_stats, stream);
}

extern "C" mi_status mi_bitlinear_gemv(const int8_t *a, int lda, const uint8_t *w_packed, void *out, int ldo,
                                       int kind, int m, int n, int k, int shift, int32_t res_mult, int res_shift,
                                       int32_t res_clamp, const float *x_scale, float w_scale, int64_t *row_stats,
                                       void *stream) {
    return bitlinear_impl("mi_bitlinear_gemv", Path::kGemv, a, lda, w_packed, out, ldo, kind, m, n, k, shift,
                          res_mult, res_shift, res_clamp, x_scale, w_scale, row_stats, stream);
}

extern "C" mi_status mi_bitlinear_residual_parts(const int8_t *a, int lda, const uint8_t *w_packed, int32_t *r,
                                                 int ldr, int m, int n, int k, int32_t res_mult, int res_shift,
                                                 int32_t res_clamp, int64_t *stats_parts, void *stream) {
    const char *fn = "mi_bitlinear_residual_parts";
    clear_error();
    mi_status st = validate(fn, a, lda, w_packed, r, ldr, MI_OUT_RESIDUAL, m, n, k, 0, res_shift, nullptr, res_clamp);
    if (st != MI_OK || (int64_t)m * n == 0) return st;
    MI_REQUIRE(m <= 64, MI_ERR_BAD_DIM, "%s: m=%d must be <= 64", fn, m);
    MI_REQUIRE(k % 64 == 0, MI_ERR_BAD_DIM, "%s: k=%d must be a multiple of 64", fn, k);
    MI_REQUIRE(stats_parts, MI_ERR_NULL_POINTER, "%s: stats_parts is required", fn);
    MI_REQUIRE(aligned(w_packed, 16) && aligned(stats_parts, 16), MI_ERR_BAD_ALIGNMENT,
               "%s: w_packed and stats_parts must be 16-byte aligned", fn);
    GemmArgs g =
        make_args(a, lda, w_packed, r, ldr, m, n, k, 0, res_mult, res_shift, nullptr, 0.0f, nullptr, res_clamp);
    g.stats_parts = stats_parts;
    if (m > 16)
        hipLaunchKernelGGL(resid_gemv16_kernel<true>, dim3((unsigned)((n + 15) / 16), (unsigned)((m + 15) / 16)),
                           dim3(512), 0, as_stream(stream), g);
    else
        hipLaunchKernelGGL(resid_gemv16_kernel<false>, dim3((unsigned)((n + 15) / 16), 1u), dim3(512), 0,
                           as_stream(stream), g);
    return check_launch(fn);
}

extern "C" mi_status mi_in_proj_conv(const int8_t *a, int lda, const uint8_t *w_in, int shift, const int8_t *conv_w,
                                     const int32_t *conv_b, const int8_t *state_in, int8_t *state_out, int8_t *xs,
                                     int8_t *xz, int ldxz, int batch, int len, int d_model, int d_inner,
                                     void *stream) {
    const char *fn = "mi_in_proj_conv";
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "%s: negative size", fn);
    // tile counts are computed as (m + kBM - 1) / kBM in int
    MI_REQUIRE((int64_t)batch * len <= INT32_MAX - kBM && (int64_t)d_inner * 2 <= INT32_MAX, MI_ERR_BAD_DIM,
               "%s: size exceeds int32", fn);
    const int m = batch * len;
    const uintptr_t sbytes = (uintptr_t)batch * 3 * (uintptr_t)d_inner;
    if (len == 0 && sbytes > 0) {
        // no rows: state_out receives state_in unchanged (zeros when state_in is NULL)
        MI_REQUIRE(state_out, MI_ERR_NULL_POINTER, "%s: state_out is required", fn);
        MI_REQUIRE(d_inner % 4 == 0 && aligned(state_out, 4) && aligned(state_in, 4), MI_ERR_BAD_ALIGNMENT,
                   "%s: the states must be 4-byte aligned and d_inner a multiple of 4", fn);
        if (state_in) {
            const uintptr_t i0 = reinterpret_cast<uintptr_t>(state_in), o0 = reinterpret_cast<uintptr_t>(state_out);
            MI_REQUIRE(i0 + sbytes <= o0 || o0 + sbytes <= i0, MI_ERR_BAD_ARG, "%s: state_in and state_out overlap",
                       fn);
        }
        const int64_t words = (int64_t)(sbytes / 4);
        hipLaunchKernelGGL(conv_state_carry_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                           as_stream(stream), reinterpret_cast<const uint32_t *>(state_in),
                           reinterpret_cast<uint32_t *>(state_out), words);
        return check_launch(fn);
    }
    mi_status st = validate(fn, a, lda, w_in, xz, ldxz, MI_OUT_INT8, m, 2 * d_inner, d_model, shift, 0, nullptr);
    if (st != MI_OK || (int64_t)m * d_inner == 0) return st;
    MI_REQUIRE(d_inner % kBN == 0, MI_ERR_BAD_DIM, "%s: d_inner=%d must be a multiple of %d", fn, d_inner, kBN);
    MI_REQUIRE(d_model % 64 == 0, MI_ERR_BAD_DIM, "%s: d_model=%d must be a multiple of 64", fn, d_model);
    MI_REQUIRE(conv_w && conv_b && state_out && xs, MI_ERR_NULL_POINTER,
               "%s: conv_w, conv_b, state_out and xs are required", fn);
    MI_REQUIRE(aligned(w_in, 16) && aligned(xz, 16) && ldxz % 16 == 0, MI_ERR_BAD_ALIGNMENT,
               "%s: w_in and xz must be 16-byte aligned and ldxz a multiple of 16", fn);
    MI_REQUIRE(aligned(conv_w, 4) && aligned(conv_b, 4) && aligned(xs, 4) && aligned(state_out, 4) &&
                   aligned(state_in, 4),
               MI_ERR_BAD_ALIGNMENT, "%s: conv_w, conv_b, xs and the states must be 4-byte aligned", fn);
    if (state_in) {
        const uintptr_t i0 = reinterpret_cast<uintptr_t>(state_in), o0 = reinterpret_cast<uintptr_t>(state_out);
        // blocks read the old state of a sequence's first rows while others
        // write the new state of its last rows: the buffers must be distinct
        MI_REQUIRE(i0 + sbytes <= o0 || o0 + sbytes <= i0, MI_ERR_BAD_ARG, "%s: state_in and state_out overlap", fn);
    }
    GemmArgs g = make_args(a, lda, w_in, xz, ldxz, m, 2 * d_inner, d_model, shift, 0, 0, nullptr, 0.0f, nullptr);
    ConvArgs cv{};
    cv.w = conv_w; cv.b = conv_b; cv.st_in = state_in; cv.st_out = state_out; cv.xs = xs;
    cv.D = d_inner; cv.L = len;
    const int64_t tiles32 = (int64_t)((m + kG2ConvRows - 1) / kG2ConvRows + (m + kG2BM - 1) / kG2BM) * (d_inner / kG2BN);
    const bool big = d_inner % kG2BN == 0 && gemm32_fits(g, tiles32);
    const int64_t nt = d_inner / (big ? kG2BN : kBN);
    const int64_t xb = (int64_t)((m + (big ? kG2ConvRows : kConvRows) - 1) / (big ? kG2ConvRows : kConvRows)) * nt;
    const int64_t zb = (int64_t)((m + kBM - 1) / kBM) * nt;   // kG2BM == kBM
    MI_REQUIRE(xb + zb <= INT32_MAX, MI_ERR_BAD_DIM, "%s: grid too large", fn);
    cv.x_blocks = (int)xb;
    if (big)
        hipLaunchKernelGGL(gemm32_conv_kernel, dim3((unsigned)(xb + zb)), dim3(256), 0, as_stream(stream), g, cv);
    else
        hipLaunchKernelGGL(gemm_conv_kernel, dim3((unsigned)(xb + zb)), dim3(256), 0, as_stream(stream), g, cv);
    return check_launch(fn);
}

extern "C" mi_status mi_pack_ternary(const int8_t *w, uint8_t *packed, int n, int k, void *stream) {
    clear_error();
    MI_REQUIRE(n >= 0 && k >= 0, MI_ERR_BAD_DIM, "mi_pack_ternary: negative size");
    MI_REQUIRE(k % 16 == 0, MI_ERR_BAD_DIM, "mi_pack_ternary: k=%d must be a multiple of 16", k);
    if ((int64_t)n * k == 0) return MI_OK;
    MI_REQUIRE(w && packed, MI_ERR_NULL_POINTER, "mi_pack_ternary: w and packed are required");
    MI_REQUIRE(aligned(packed, 4), MI_ERR_BAD_ALIGNMENT, "mi_pack_ternary: packed must be 4-byte aligned");
    const int64_t words = (int64_t)n * (k / 16);
    hipLaunchKernelGGL(pack_ternary_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, as_stream(stream), w,
                       reinterpret_cast<uint32_t *>(packed), words, k / 16);
    return check_launch("mi_pack_ternary");
}

extern "C" mi_status mi_act_quant_f32(const float *x, int8_t *xq, float *x_scale, int m, int k, void *stream) {
    clear_error();
    MI_REQUIRE(m >= 0 && k >= 0, MI_ERR_BAD_DIM, "mi_act_quant_f32: negative size");
    if (m == 0) return MI_OK;
    MI_REQUIRE(k > 0, MI_ERR_BAD_DIM, "mi_act_quant_f32: k must be positive");
    MI_REQUIRE(x && xq && x_scale, MI_ERR_NULL_POINTER, "mi_act_quant_f32: x, xq and x_scale are required");
    hipLaunchKernelGGL(act_quant_kernel, dim3((unsigned)m), dim3(256), 0, as_stream(stream), x, xq, x_scale, k);
    return check_launch("mi_act_quant_f32");
}
