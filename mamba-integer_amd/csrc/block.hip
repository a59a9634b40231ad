// Elementwise and row stages of the integer Mamba block on gfx950 (spec
// mi-spec-2, rules 4.1, 4.3-4.4 and the model's embedding / greedy pick).
#include "mi_mfma.hpp"

namespace mi {
namespace {

// ------------------------------------------------------------ BitShiftNorm
// One block per token.  The row is read once into registers; the mean and the
// sum of squares are exact int64 block reductions.
constexpr int kNormThreads = 256;
constexpr int kNormMaxPer = 32;  // dim <= 8192

__device__ int64_t block_sum64(int64_t v, int64_t *red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    int64_t t = 0;
    for (int w = 0; w < kNormThreads / 64; ++w) t += red[w];
    __syncthreads();
    return t;
}

// V2: the threshold table of BitShiftNormV2 (spec rule 7.1) instead of 4.1.
template <bool V2>
__global__ __launch_bounds__(kNormThreads) void norm_kernel(const int32_t *r, const int16_t *gamma, int8_t *out,
                                                            int dim) {
    __shared__ int64_t red[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const int32_t *rr = r + row * dim;
    int32_t v[kNormMaxPer];
    int64_t s = 0;
    for (int j = 0; j < kNormMaxPer; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        v[j] = i < dim ? rr[i] : 0;
        s += v[j];
    }
    const int64_t sum = block_sum64(s, red);
    const int64_t mu = sum >= 0 ? sum / dim : -((-sum + dim - 1) / dim);  // floor
    int64_t q = 0;
    for (int j = 0; j < kNormMaxPer; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        if (i < dim) {
            const int64_t x = v[j] - mu;
            q += x * x;
        }
    }
    const int64_t S = block_sum64(q, red);
    // threshold table of _find_power_of_2_scale (mamba_integer_model.py:169-182)
    // on var = S / (dim * 2^16): k = #[var >= 4^j, j=1..8] - #[var < 4^-j, j=1..3]
    // (V2: j=1..6 and j=1..2); norm_shift_for takes the statistics, so S is
    // passed as s2 with s1 = 0 about the already-subtracted mean
    int64_t zero_mu;
    const int sh = norm_shift_for<V2>(0, S, dim, &zero_mu);
    for (int j = 0; j < kNormMaxPer; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        if (i < dim) out[row * dim + i] = (int8_t)clamp64(rshr64((int64_t)(v[j] - mu) * gamma[i], sh), -127, 127);
    }
}

// One wave per row, one pass: the row stays in registers (16 int4 per lane,
// dim <= 4096) while its sum and sum of squares are reduced.
constexpr int kNormWaveMax = 16;

template <bool V2>
__global__ __launch_bounds__(256) void norm_wave_kernel(const int32_t *r, const int16_t *gamma, int8_t *out,
                                                        int tokens, int dim) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= tokens) return;
    const int32_t *rr = r + row * dim;
    int4 v[kNormWaveMax];
    int64_t s1 = 0, s2 = 0;
#pragma unroll
    for (int j = 0; j < kNormWaveMax; ++j) {
        const int i = 4 * lane + 256 * j;
        v[j] = i < dim ? *reinterpret_cast<const int4 *>(rr + i) : make_int4(0, 0, 0, 0);
        s1 += (int64_t)v[j].x + v[j].y + v[j].z + v[j].w;
        s2 += (int64_t)v[j].x * v[j].x + (int64_t)v[j].y * v[j].y + (int64_t)v[j].z * v[j].z +
              (int64_t)v[j].w * v[j].w;
    }
    for (int off = 32; off > 0; off >>= 1) {
        s1 += __shfl_xor(s1, off);
        s2 += __shfl_xor(s2, off);
    }
    int64_t mu;
    const int sh = norm_shift_for<V2>(s1, s2, dim, &mu);
#pragma unroll
    for (int j = 0; j < kNormWaveMax; ++j) {
        const int i = 4 * lane + 256 * j;
        if (i < dim) {
            const int vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            uint32_t o = 0;
            for (int q = 0; q < 4; ++q)
                o |= (uint32_t)((int)clamp64(rshr64((int64_t)(vv[q] - mu) * gamma[i + q], sh), -127, 127) & 255)
                     << (8 * q);
            *reinterpret_cast<uint32_t *>(out + row * dim + i) = o;
        }
    }
}

// norm_wave_kernel for dim = 256 * J: every load unconditional and issued up
// front (the row's J int4 per lane and its gains as one 8-byte load per 4
// channels), so the wave waits once instead of once per conditional load.
template <bool V2, int J>
__global__ __launch_bounds__(256) void norm_wave_fixed_kernel(const int32_t *r, const int16_t *gamma, int8_t *out,
                                                              int tokens) {
    constexpr int dim = 256 * J;
    const int lane = threadIdx.x & 63;
    const int64_t row = min((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6), (int64_t)tokens - 1);
    const int32_t *rr = r + row * dim;
    int4 v[J];
    int2 gv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) v[j] = *reinterpret_cast<const int4 *>(rr + 4 * lane + 256 * j);
#pragma unroll
    for (int j = 0; j < J; ++j) gv[j] = *reinterpret_cast<const int2 *>(gamma + 4 * lane + 256 * j);
    int64_t s1 = 0, s2 = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        s1 += (int64_t)v[j].x + v[j].y + v[j].z + v[j].w;
        s2 += (int64_t)v[j].x * v[j].x + (int64_t)v[j].y * v[j].y + (int64_t)v[j].z * v[j].z +
              (int64_t)v[j].w * v[j].w;
    }
    for (int off = 32; off > 0; off >>= 1) {
        s1 += __shfl_xor(s1, off);
        s2 += __shfl_xor(s2, off);
    }
    int64_t mu;
    const int sh = norm_shift_for<V2>(s1, s2, dim, &mu);
    if ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6) >= tokens) return;  // the clamped duplicate row
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        const int gg[4] = {(int)(int16_t)gv[j].x, gv[j].x >> 16, (int)(int16_t)gv[j].y, gv[j].y >> 16};
        uint32_t o = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o |= (uint32_t)((int)clamp64(rshr64((int64_t)(vv[q] - mu) * gg[q], sh), -127, 127) & 255) << (8 * q);
        *reinterpret_cast<uint32_t *>(out + row * dim + 4 * lane + 256 * j) = o;
    }
}

template <bool V2>
bool launch_norm_wave_fixed(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens, int dim,
                            hipStream_t st) {
    if (dim % 256 != 0 || !aligned(gamma, 8)) return false;
    const dim3 grid((unsigned)((tokens + 3) / 4));
    switch (dim / 256) {
#define MI_NWCASE(JJ)                                                                                      \
    case JJ:                                                                                               \
        hipLaunchKernelGGL((norm_wave_fixed_kernel<V2, JJ>), grid, dim3(256), 0, st, r, gamma, out, tokens); \
        return true;
        MI_NWCASE(1)
        MI_NWCASE(2)
        MI_NWCASE(3)
        MI_NWCASE(4)
        MI_NWCASE(6)
        MI_NWCASE(8)
        MI_NWCASE(12)
        MI_NWCASE(16)
#undef MI_NWCASE
    }
    return false;
}

// --------------------------------------------------------------- embedding
__global__ void embed_kernel(const int64_t *ids, const int8_t *emb, int32_t *r, int tokens, int dim, int vocab) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)tokens * dim) return;
    const int64_t t = i / dim;
    const int c = (int)(i % dim);
    const int64_t id = ids[t];
    // an id outside [0, vocab) reads as a zero row instead of faulting
    r[i] = (id >= 0 && id < vocab) ? (int32_t)emb[id * dim + c] * 16 : 0;
}

// One block per token: r = emb[id] << 4, its row statistics into
// stats[0][t] = (sum r, sum r^2), and stats[j][t] = 0 for the later layers
// (their out_proj epilogues accumulate into them).
__global__ __launch_bounds__(256) void embed_stats_kernel(const int64_t *ids, const int8_t *emb, int32_t *r,
                                                          int tokens, int dim, int vocab, int64_t *stats,
                                                          int stats_layers) {
    __shared__ int64_t red[2][4];
    const int64_t t = blockIdx.x;
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    int64_t s1 = 0, s2 = 0;
    for (int c = threadIdx.x; c < dim; c += 256) {
        const int32_t v = ok ? (int32_t)emb[id * dim + c] * 16 : 0;
        r[t * dim + c] = v;
        s1 += v;
        s2 += (int64_t)v * v;
    }
    for (int off = 32; off > 0; off >>= 1) {
        s1 += __shfl_xor(s1, off);
        s2 += __shfl_xor(s2, off);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wave] = s1;
        red[1][wave] = s2;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        stats[2 * t] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
        stats[2 * t + 1] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    }
    for (int j = 1 + (int)threadIdx.x; j < stats_layers; j += 256) {
        stats[((int64_t)j * tokens + t) * 2] = 0;
        stats[((int64_t)j * tokens + t) * 2 + 1] = 0;
    }
}

// Greedy pick of row t from per-block partial keys (logit << 32 | 0x7FFFFFFF -
// index): the largest key, decoded to its index, returned to every thread.
__device__ int64_t block_pick(const int64_t *keys, int nkeys) {
    __shared__ int64_t s_best[4];
    int64_t best = INT64_MIN;
    for (int i = threadIdx.x; i < nkeys; i += 256) best = max(best, keys[i]);
    for (int off = 32; off > 0; off >>= 1) best = max(best, (int64_t)__shfl_xor(best, off));
    if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
    __syncthreads();
    best = max(max(s_best[0], s_best[1]), max(s_best[2], s_best[3]));
    return 0x7FFFFFFF - (int64_t)(uint32_t)(best & 0xFFFFFFFF);
}

__global__ __launch_bounds__(256) void argmax_keys_kernel(const int64_t *keys, int nkeys, int64_t *ids) {
    const int64_t t = blockIdx.x;
    const int64_t id = block_pick(keys + t * nkeys, nkeys);
    if (threadIdx.x == 0) ids[t] = id;
}

// Greedy pick of the previous step's logits, then the embedding row of the
// picked id with its row statistics (embed_stats_kernel of that id).
__global__ __launch_bounds__(256) void embed_argmax_kernel(const int64_t *keys, int nkeys, int64_t *ids,
                                                           const int8_t *emb, int32_t *r, int tokens, int dim,
                                                           int vocab, int64_t *stats, int stats_layers) {
    __shared__ int64_t red[2][4];
    const int64_t t = blockIdx.x;
    const int64_t id = block_pick(keys + t * nkeys, nkeys);
    if (threadIdx.x == 0) ids[t] = id;
    const bool ok = id >= 0 && id < vocab;
    int64_t s1 = 0, s2 = 0;
    for (int c = threadIdx.x; c < dim; c += 256) {
        const int32_t v = ok ? (int32_t)emb[id * dim + c] * 16 : 0;
        r[t * dim + c] = v;
        s1 += v;
        s2 += (int64_t)v * v;
    }
    for (int off = 32; off > 0; off >>= 1) {
        s1 += __shfl_xor(s1, off);
        s2 += __shfl_xor(s2, off);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wave] = s1;
        red[1][wave] = s2;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        stats[2 * t] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
        stats[2 * t + 1] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    }
    for (int j = 1 + (int)threadIdx.x; j < stats_layers; j += 256) {
        stats[((int64_t)j * tokens + t) * 2] = 0;
        stats[((int64_t)j * tokens + t) * 2 + 1] = 0;
    }
}

// Elementwise BitShiftNorm from precomputed row statistics: thread = 4 channels.
template <bool V2>
__global__ __launch_bounds__(256) void norm_stats_kernel(const int32_t *r, const int16_t *gamma, int8_t *out,
                                                         const int64_t *stats, int tokens, int dim) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int d4 = dim / 4;
    if (i >= (int64_t)tokens * d4) return;
    const int64_t t = i / d4;
    const int c = (int)(i % d4) * 4;
    int64_t mu;
    const int sh = norm_shift_for<V2>(stats[2 * t], stats[2 * t + 1], dim, &mu);
    const int4 v = *reinterpret_cast<const int4 *>(r + t * dim + c);
    const int vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t o = 0;
    for (int q = 0; q < 4; ++q)
        o |= (uint32_t)((int)clamp64(rshr64((int64_t)(vv[q] - mu) * gamma[c + q], sh), -127, 127) & 255) << (8 * q);
    *reinterpret_cast<uint32_t *>(out + t * dim + c) = o;
}

// BitShiftNorm from per-block row-statistics partials (int64 [tokens][nparts][2],
// the stores of mi_bitlinear_residual_parts): block (c, t) loads its 1024
// channels of row t, sums the row's nparts pairs across the block, then
// normalizes 4 channels per thread.
template <bool V2>
__global__ __launch_bounds__(256) void norm_parts_kernel(const int32_t *r, const int16_t *gamma, int8_t *out,
                                                         const int64_t *parts, int nparts, int dim) {
    __shared__ int64_t red[2][4];
    const int64_t t = blockIdx.y;
    const int c = (blockIdx.x * 256 + (int)threadIdx.x) * 4;
    const bool ok = c < dim;
    const int4 v = *reinterpret_cast<const int4 *>(r + t * dim + (ok ? c : 0));
    const v2l *pp = reinterpret_cast<const v2l *>(parts + t * nparts * 2);
    int64_t s1 = 0, s2 = 0;
    for (int i = threadIdx.x; i < nparts; i += 256) {
        const v2l p = pp[i];
        s1 += p[0];
        s2 += p[1];
    }
    for (int off = 32; off > 0; off >>= 1) {
        s1 += __shfl_xor(s1, off);
        s2 += __shfl_xor(s2, off);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wave] = s1;
        red[1][wave] = s2;
    }
    __syncthreads();
    s1 = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    s2 = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    if (!ok) return;
    int64_t mu;
    const int sh = norm_shift_for<V2>(s1, s2, dim, &mu);
    const int vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t o = 0;
    for (int q = 0; q < 4; ++q)
        o |= (uint32_t)((int)clamp64(rshr64((int64_t)(vv[q] - mu) * gamma[c + q], sh), -127, 127) & 255) << (8 * q);
    *reinterpret_cast<uint32_t *>(out + t * dim + c) = o;
}

// ----------------------------------------------------- conv + squareplus
constexpr int kConvTT = 16;  // time steps per thread

// Thread = (b, group of kConvTT steps, 4 channels).  The thread of step-group 0
// owns the conv state of its channels: it reads state_in and writes state_out
// (from the inputs x[L-3..L-1], which no thread modifies), so in-place state
// updates are race free.
__global__ __launch_bounds__(256) void conv_sqp_kernel(const int8_t *xz, int64_t xz_stride, const int8_t *w,
                                                       const int32_t *bias, const int8_t *st_in, int8_t *st_out,
                                                       int8_t *xs, int B, int L, int D) {
    const int D4 = D / 4;
    const int TG = (L + kConvTT - 1) / kConvTT;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * TG * D4) return;
    const int d4 = (int)(i % D4);
    const int tg = (int)((i / D4) % TG);
    const int b = (int)(i / ((int64_t)D4 * TG));
    const int d = d4 * 4;

    int wv[4][4], bv[4];
    for (int c = 0; c < 4; ++c) {
        const uint32_t ww = *reinterpret_cast<const uint32_t *>(w + (int64_t)(d + c) * 4);
        for (int j = 0; j < 4; ++j) wv[c][j] = (int)(int8_t)(ww >> (8 * j));
        bv[c] = bias[d + c];
    }
    auto xrow = [&](int t) -> uint32_t {  // 4 channels of x at time t (t may be < 0: conv state)
        if (t >= 0) return *reinterpret_cast<const uint32_t *>(xz + ((int64_t)b * L + t) * xz_stride + d);
        if (!st_in) return 0u;
        return *reinterpret_cast<const uint32_t *>(st_in + ((int64_t)b * 3 + (3 + t)) * D + d);
    };
    const int t0 = tg * kConvTT;
    const int t1 = min(L, t0 + kConvTT);
    uint32_t win[3] = {xrow(t0 - 3), xrow(t0 - 2), xrow(t0 - 1)};
    uint32_t keep_state[3] = {win[0], win[1], win[2]};  // x[-3..-1] for the state update when L < 3
    for (int t = t0; t < t1; ++t) {
        const uint32_t cur = xrow(t);
        uint32_t o = 0;
        for (int c = 0; c < 4; ++c) {
            int32_t acc = bv[c];
            acc += wv[c][0] * (int)(int8_t)(win[0] >> (8 * c));
            acc += wv[c][1] * (int)(int8_t)(win[1] >> (8 * c));
            acc += wv[c][2] * (int)(int8_t)(win[2] >> (8 * c));
            acc += wv[c][3] * (int)(int8_t)(cur >> (8 * c));
            o |= (uint32_t)(sqp_q(acc) & 255) << (8 * c);
        }
        *reinterpret_cast<uint32_t *>(xs + ((int64_t)b * L + t) * D + d) = o;
        win[0] = win[1];
        win[1] = win[2];
        win[2] = cur;
    }
    if (tg == 0 && st_out) {
        for (int j = 0; j < 3; ++j) {
            const int t = L - 3 + j;
            // keep_state is selected, not indexed: a register array indexed at
            // run time would be kept in scratch
            const uint32_t kept = t == -3 ? keep_state[0] : (t == -2 ? keep_state[1] : keep_state[2]);
            const uint32_t val =
                t >= 0 ? *reinterpret_cast<const uint32_t *>(xz + ((int64_t)b * L + t) * xz_stride + d) : kept;
            *reinterpret_cast<uint32_t *>(st_out + ((int64_t)b * 3 + j) * D + d) = val;
        }
    }
}

// ---------------------------------------------------------------- argmax
// One block per row.  Each thread walks its columns in increasing order with
// four independent 16-byte loads in flight, keeping the first maximum; the
// block reduction prefers the larger value, then the smaller index.
__global__ __launch_bounds__(256) void argmax_kernel(const int32_t *logits, int64_t ld, int64_t *out, int cols,
                                                     bool vec) {
    __shared__ int32_t sv[256];
    __shared__ int32_t si[256];
    const int64_t row = blockIdx.x;
    const int32_t *lr = logits + row * ld;
    int32_t best = INT32_MIN;
    int32_t bi = 0x7fffffff;
    int cstart = 0;
    if (vec) {
        const int nv = cols / 4;
        const int4 *lv = reinterpret_cast<const int4 *>(lr);
        for (int v0 = threadIdx.x; v0 < nv; v0 += 1024) {
            int4 q[4];
            for (int u = 0; u < 4; ++u) {
                const int v = v0 + 256 * u;
                q[u] = v < nv ? lv[v] : make_int4(INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN);
            }
            for (int u = 0; u < 4; ++u) {
                const int c = 4 * (v0 + 256 * u);
                if (q[u].x > best) { best = q[u].x; bi = c; }
                if (q[u].y > best) { best = q[u].y; bi = c + 1; }
                if (q[u].z > best) { best = q[u].z; bi = c + 2; }
                if (q[u].w > best) { best = q[u].w; bi = c + 3; }
            }
        }
        cstart = 4 * nv;
    }
    for (int c = cstart + threadIdx.x; c < cols; c += 256) {
        const int32_t v = lr[c];
        if (v > best || (v == best && c < bi)) { best = v; bi = c; }
    }
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const int32_t v2 = sv[threadIdx.x + s], i2 = si[threadIdx.x + s];
            if (v2 > sv[threadIdx.x] || (v2 == sv[threadIdx.x] && i2 < si[threadIdx.x])) {
                sv[threadIdx.x] = v2;
                si[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[row] = si[0];
}

}  // namespace
}  // namespace mi

using namespace mi;

namespace mi {
namespace {
template <bool V2>
mi_status bitshift_norm_impl(const char *fn, const int32_t *r, const int16_t *gamma, int8_t *out, int tokens, int dim,
                             const int64_t *row_stats, void *stream) {
    clear_error();
    MI_REQUIRE(tokens >= 0, MI_ERR_BAD_DIM, "%s: negative tokens", fn);
    MI_REQUIRE(dim >= 1 && dim <= kNormThreads * kNormMaxPer, MI_ERR_BAD_DIM, "%s: dim=%d outside [1,%d]", fn, dim,
               kNormThreads * kNormMaxPer);
    if (tokens == 0) return MI_OK;
    MI_REQUIRE(r && gamma && out, MI_ERR_NULL_POINTER, "%s: r, gamma and out are required", fn);
    if (row_stats) {
        MI_REQUIRE(dim % 4 == 0 && aligned(r, 16) && aligned(out, 4), MI_ERR_BAD_ALIGNMENT,
                   "%s: with row_stats, dim %% 4 == 0 and aligned r/out are required", fn);
        const int64_t threads = (int64_t)tokens * (dim / 4);
        hipLaunchKernelGGL(norm_stats_kernel<V2>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                           as_stream(stream), r, gamma, out, row_stats, tokens, dim);
    } else if (dim % 4 == 0 && dim <= 256 * kNormWaveMax && aligned(r, 16) && aligned(out, 4)) {
        if (!launch_norm_wave_fixed<V2>(r, gamma, out, tokens, dim, as_stream(stream)))
            hipLaunchKernelGGL(norm_wave_kernel<V2>, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0,
                               as_stream(stream), r, gamma, out, tokens, dim);
    } else {
        hipLaunchKernelGGL(norm_kernel<V2>, dim3((unsigned)tokens), dim3(kNormThreads), 0, as_stream(stream), r, gamma,
                           out, dim);
    }
    return check_launch(fn);
}
}  // namespace
}  // namespace mi

extern "C" mi_status mi_bitshift_norm(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens, int dim,
                                      const int64_t *row_stats, void *stream) {
    return bitshift_norm_impl<false>("mi_bitshift_norm", r, gamma, out, tokens, dim, row_stats, stream);
}

extern "C" mi_status mi_bitshift_norm_v2(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens, int dim,
                                         const int64_t *row_stats, void *stream) {
    return bitshift_norm_impl<true>("mi_bitshift_norm_v2", r, gamma, out, tokens, dim, row_stats, stream);
}

extern "C" mi_status mi_bitshift_norm_parts(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens,
                                            int dim, const int64_t *stats_parts, int nparts, int v2, void *stream) {
    clear_error();
    MI_REQUIRE(tokens >= 0 && tokens <= 65535, MI_ERR_BAD_DIM,
               "mi_bitshift_norm_parts: tokens=%d outside [0,65535] (the grid's y dimension)", tokens);
    MI_REQUIRE(dim >= 4 && dim % 4 == 0 && dim <= 65536, MI_ERR_BAD_DIM,
               "mi_bitshift_norm_parts: dim=%d must be a multiple of 4 in [4,65536]", dim);
    MI_REQUIRE(nparts >= 1, MI_ERR_BAD_ARG, "mi_bitshift_norm_parts: nparts=%d must be >= 1", nparts);
    if (tokens == 0) return MI_OK;
    MI_REQUIRE(r && gamma && out && stats_parts, MI_ERR_NULL_POINTER,
               "mi_bitshift_norm_parts: r, gamma, out and stats_parts are required");
    MI_REQUIRE(aligned(r, 16) && aligned(out, 4) && aligned(stats_parts, 16), MI_ERR_BAD_ALIGNMENT,
               "mi_bitshift_norm_parts: r and stats_parts 16-byte, out 4-byte aligned");
    const dim3 grid((unsigned)((dim + 1023) / 1024), (unsigned)tokens);
    if (v2)
        hipLaunchKernelGGL(norm_parts_kernel<true>, grid, dim3(256), 0, as_stream(stream), r, gamma, out, stats_parts,
                           nparts, dim);
    else
        hipLaunchKernelGGL(norm_parts_kernel<false>, grid, dim3(256), 0, as_stream(stream), r, gamma, out,
                           stats_parts, nparts, dim);
    return check_launch("mi_bitshift_norm_parts");
}

extern "C" mi_status mi_embed(const int64_t *ids, const int8_t *emb, int32_t *r, int tokens, int dim, int vocab,
                              int64_t *row_stats, int stats_layers, void *stream) {
    clear_error();
    MI_REQUIRE(tokens >= 0 && dim >= 0 && vocab >= 0, MI_ERR_BAD_DIM, "mi_embed: negative size");
    if ((int64_t)tokens * dim == 0) return MI_OK;
    MI_REQUIRE(ids && emb && r, MI_ERR_NULL_POINTER, "mi_embed: ids, emb and r are required");
    if (row_stats) {
        MI_REQUIRE(stats_layers >= 1, MI_ERR_BAD_ARG, "mi_embed: stats_layers=%d must be >= 1", stats_layers);
        hipLaunchKernelGGL(embed_stats_kernel, dim3((unsigned)tokens), dim3(256), 0, as_stream(stream), ids, emb, r,
                           tokens, dim, vocab, row_stats, stats_layers);
        return check_launch("mi_embed");
    }
    const int64_t n = (int64_t)tokens * dim;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), ids, emb, r,
                       tokens, dim, vocab);
    return check_launch("mi_embed");
}

extern "C" mi_status mi_conv_squareplus(const int8_t *xz, int xz_stride, const int8_t *conv_w, const int32_t *conv_b,
                                        const int8_t *state_in, int8_t *state_out, int8_t *xs, int batch, int len,
                                        int d_inner, void *stream) {
    clear_error();
    MI_REQUIRE(batch >= 0 && len >= 0 && d_inner >= 0, MI_ERR_BAD_DIM, "mi_conv_squareplus: negative size");
    MI_REQUIRE(d_inner % 4 == 0, MI_ERR_BAD_DIM, "mi_conv_squareplus: d_inner=%d must be a multiple of 4", d_inner);
    MI_REQUIRE(xz_stride >= d_inner && xz_stride % 4 == 0, MI_ERR_BAD_ALIGNMENT,
               "mi_conv_squareplus: xz_stride=%d must be >= d_inner and a multiple of 4", xz_stride);
    if ((int64_t)batch * d_inner == 0 || len == 0) {
        MI_REQUIRE(!state_out || state_out == state_in, MI_ERR_BAD_ARG,
                   "mi_conv_squareplus: len=0 leaves state_out unwritten; pass state_out == state_in");
        return MI_OK;
    }
    MI_REQUIRE(xz && conv_w && conv_b && xs, MI_ERR_NULL_POINTER, "mi_conv_squareplus: xz, conv_w, conv_b, xs required");
    MI_REQUIRE(aligned(xz, 4) && aligned(conv_w, 4) && aligned(xs, 4) && aligned(state_in, 4) && aligned(state_out, 4),
               MI_ERR_BAD_ALIGNMENT, "mi_conv_squareplus: pointers must be 4-byte aligned");
    const int64_t threads = (int64_t)batch * ((len + kConvTT - 1) / kConvTT) * (d_inner / 4);
    hipLaunchKernelGGL(conv_sqp_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, as_stream(stream), xz,
                       (int64_t)xz_stride, conv_w, conv_b, state_in, state_out, xs, batch, len, d_inner);
    return check_launch("mi_conv_squareplus");
}

extern "C" mi_status mi_argmax_i32(const int32_t *logits, int ld, int64_t *out, int rows, int cols, void *stream) {
    clear_error();
    MI_REQUIRE(rows >= 0 && cols >= 0, MI_ERR_BAD_DIM, "mi_argmax_i32: negative size");
    MI_REQUIRE(ld >= cols, MI_ERR_BAD_DIM, "mi_argmax_i32: ld=%d < cols=%d", ld, cols);
    if (rows == 0) return MI_OK;
    MI_REQUIRE(cols >= 1, MI_ERR_BAD_DIM, "mi_argmax_i32: cols must be positive");
    MI_REQUIRE(logits && out, MI_ERR_NULL_POINTER, "mi_argmax_i32: logits and out are required");
    const bool vec = ld % 4 == 0 && aligned(logits, 16);
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), logits, (int64_t)ld, out,
                       cols, vec);
    return check_launch("mi_argmax_i32");
}

extern "C" mi_status mi_argmax_keys(const int64_t *keys, int nkeys, int64_t *ids, int rows, void *stream) {
    clear_error();
    MI_REQUIRE(rows >= 0 && nkeys >= 1, MI_ERR_BAD_DIM, "mi_argmax_keys: rows=%d, nkeys=%d", rows, nkeys);
    if (rows == 0) return MI_OK;
    MI_REQUIRE(keys && ids, MI_ERR_NULL_POINTER, "mi_argmax_keys: keys and ids are required");
    hipLaunchKernelGGL(argmax_keys_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), keys, nkeys, ids);
    return check_launch("mi_argmax_keys");
}

extern "C" mi_status mi_embed_argmax(const int64_t *keys, int nkeys, int64_t *ids, const int8_t *emb, int32_t *r,
                                     int tokens, int dim, int vocab, int64_t *row_stats, int stats_layers,
                                     void *stream) {
    clear_error();
    MI_REQUIRE(tokens >= 0 && dim >= 0 && vocab >= 0 && nkeys >= 1, MI_ERR_BAD_DIM, "mi_embed_argmax: bad size");
    if ((int64_t)tokens * dim == 0) return MI_OK;
    MI_REQUIRE(keys && ids && emb && r && row_stats, MI_ERR_NULL_POINTER,
               "mi_embed_argmax: keys, ids, emb, r and row_stats are required");
    MI_REQUIRE(stats_layers >= 1, MI_ERR_BAD_ARG, "mi_embed_argmax: stats_layers=%d must be >= 1", stats_layers);
    hipLaunchKernelGGL(embed_argmax_kernel, dim3((unsigned)tokens), dim3(256), 0, as_stream(stream), keys, nkeys, ids,
                       emb, r, tokens, dim, vocab, row_stats, stats_layers);
    return check_launch("mi_embed_argmax");
}
