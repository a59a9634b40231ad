/*
 * mi_oracle.c — CPU restatement of the integer Mamba inference path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the test oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (libmamba_int.so) never links, calls or falls back to it.
 *
 * Every function states the rule it follows (spec version mi-spec-2) and the
 * reference file:line it restates. The integer rules the reference leaves
 * undefined (saturation, rounding, packing, the integer norm, squareplus, dt
 * and gate) are frozen in SPEC.md of this repository; the code below is the
 * executable form of those rules, written for clarity (plain int64
 * arithmetic, no tricks), with OpenMP over independent lanes.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MO_VERSION "mi-spec-2 oracle 2"

static int g_threads = 1;
/* Mutation switch for the tests that show the pins catch a planted mistake.
 * 0 = faithful. Any other value changes one rule (see mo_set_mutation). */
static int g_mutation = 0;

const char *mo_version(void) { return MO_VERSION; }

void mo_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int mo_get_threads(void) { return g_threads; }

/* 1: scan rounds to nearest instead of flooring; 2: scan drops the input
 * term's sign (uses |u|); 3: y saturates partial sums per state instead of
 * once; 4: pack swaps the +1/-1 codes; 5: norm truncates the mean; 6: gemm
 * swaps weights 0 and 3 of every group of four; 7 / 8: the float-compat scan
 * rounds / floors x * 2^sb instead of truncating; 9: the float-compat scan's
 * shift rounds instead of flooring. */
void mo_set_mutation(int m) { g_mutation = m; }

/* ---------------------------------------------------------------- helpers */
static inline int64_t floor_shr(int64_t v, int s) {
    /* arithmetic shift == floor division by 2^s (gcc/clang on two's complement) */
    return v >> s;
}
static inline int64_t rshr(int64_t v, int s) {
    return s <= 0 ? v : ((v + ((int64_t)1 << (s - 1))) >> s);
}
static inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
static inline int32_t sat32(int64_t v) { return (int32_t)clamp64(v, INT32_MIN, INT32_MAX); }
static inline int8_t sat8(int64_t v) { return (int8_t)clamp64(v, -127, 127); }
#define R_LIM ((int64_t)8388607) /* 2^23 - 1 */
static inline int32_t satR(int64_t v) { return (int32_t)clamp64(v, -R_LIM, R_LIM); }

uint64_t mo_isqrt(uint64_t v) {
    /* exact floor(sqrt(v)) by the bitwise (digit-by-digit) method */
    uint64_t res = 0, bit = (uint64_t)1 << 62;
    while (bit > v) bit >>= 2;
    while (bit) {
        if (v >= res + bit) {
            v -= res + bit;
            res = (res >> 1) + bit;
        } else {
            res >>= 1;
        }
        bit >>= 2;
    }
    return res;
}

/* One recurrence step (dyadic_mamba_kernel.cu:53-59): h*num exact, arithmetic
 * shift (floor), add input, saturate to int32 (spec rule 1). */
static inline int32_t scan_step(int32_t h, int32_t n, int k, int64_t u) {
    int64_t p = (int64_t)h * (int64_t)n;
    int64_t d;
    if (g_mutation == 1)
        d = rshr(p, k);
    else
        d = floor_shr(p, k);
    if (g_mutation == 2) u = u < 0 ? -u : u;
    return sat32(d + u);
}

/* --------------------------------------------- 1. dyadic selective scan */
/* Config-1 layout: x[B,L,D] i8, Bm/Cm[B,L,N] i8, ndec[D,N] i32 (time
 * invariant), y[B,L,D] i32, hstate[B,D,N] i32 (nullable: zero start, final
 * state not returned).  Restates the integer core of dyadic_scan_kernel
 * (dyadic_mamba_kernel.cu:35-63) over the selective-scan dataflow of
 * MambaIntegerBlock.forward (mamba_integer_model.py:428-440). */
int mo_dyadic_scan(const int8_t *x, const int8_t *Bm, const int8_t *Cm, const int32_t *ndec,
                   int k, int32_t *y, int32_t *hstate, int B, int L, int D, int N) {
    if (N > 1024) return 2;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d = 0; d < D; ++d) {
            int32_t h[1024];
            for (int n = 0; n < N; ++n)
                h[n] = hstate ? hstate[((int64_t)b * D + d) * N + n] : 0;
            for (int t = 0; t < L; ++t) {
                int64_t bt = (int64_t)b * L + t;
                int64_t xv = x[bt * D + d];
                int64_t acc = 0;
                for (int n = 0; n < N; ++n) {
                    h[n] = scan_step(h[n], ndec[(int64_t)d * N + n], k, (int64_t)Bm[bt * N + n] * xv);
                    int64_t term = (int64_t)Cm[bt * N + n] * h[n];
                    if (g_mutation == 3)
                        acc = sat32(acc + term);
                    else
                        acc += term;
                }
                y[bt * D + d] = sat32(acc);
            }
            if (hstate)
                for (int n = 0; n < N; ++n) hstate[((int64_t)b * D + d) * N + n] = h[n];
        }
    }
    return 0;
}

/* Float-compat form of the reference kernel launch_dyadic_scan
 * (dyadic_mamba_kernel.cu:8-67,134-153): x/h fp32 [B,S,D], nums/shifts int32
 * [B,S,D]; x_fixed = (long long)(x * 2^sb) (fp32 product, truncation), int64
 * state, h = (h*num) >> shift, h += x_fixed, out = (float)h / 2^sb. */
void mo_dyadic_scan_f32(const float *x, const int32_t *nums, const int32_t *shifts, float *hout,
                        int B, int S, int D, int sb) {
    const float scale_f = (float)((long long)1 << sb);
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d = 0; d < D; ++d) {
            long long h = 0;
            for (int t = 0; t < S; ++t) {
                int64_t off = ((int64_t)b * S + t) * D + d;
                float xs = x[off] * scale_f;
                long long xf = (long long)xs;
                if (g_mutation == 7) xf = llroundf(xs);          /* planted: round, not truncate */
                if (g_mutation == 8) xf = (long long)floorf(xs); /* planted: floor, not truncate */
                h = h * (long long)nums[off];
                if (g_mutation == 9 && shifts[off] > 0)          /* planted: rounding shift */
                    h += (long long)1 << (shifts[off] - 1);
                h = h >> shifts[off];
                h += xf;
                hout[off] = (float)h / scale_f;
            }
        }
    }
}

/* Elementwise integer form of DyadicScanFunction.apply(u, nums, shifts)
 * (mamba_integer_model.py:260-316 interface; integer rule of
 * dyadic_mamba_kernel.cu:53-59): u/n int32 [B,L,C], one shift k, h int32
 * [B,L,C]; hstate [B,C] nullable in/out. */
void mo_dyadic_scan_elementwise(const int32_t *u, const int32_t *n, int k, int32_t *h,
                                int32_t *hstate, int B, int L, int C) {
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int c = 0; c < C; ++c) {
            int32_t s = hstate ? hstate[(int64_t)b * C + c] : 0;
            for (int t = 0; t < L; ++t) {
                int64_t off = ((int64_t)b * L + t) * C + c;
                s = scan_step(s, n[off], k, u[off]);
                h[off] = s;
            }
            if (hstate) hstate[(int64_t)b * C + c] = s;
        }
    }
}

/* Chunked elementwise scan with the outputs of ssd_chunked_scan_forward
 * (ssd_chunked_scan.py:382-422; chunk loop of ssd_intra_chunk_matmul_kernel,
 * :346-379): h[t] = sat32(floor(h[t-1]*n[t] / 2^k) + u[t]) per (b, channel)
 * over u, n int32 [B,L,C]; final_h[B,nc,C] (nullable) is h at the last step of
 * every chunk of cs steps; decay_to_end[B,nc,C] (nullable) is the chunk's
 * cumulative decay prod n[t]/2^k in Q30, rounded down after every step:
 * p = 2^30, p = sat32(floor(p*n[t] / 2^k)) over the chunk's steps.
 * hstate[B,C] nullable in/out. */
void mo_dyadic_chunked_scan(const int32_t *u, const int32_t *n, int k, int cs, int32_t *h, int32_t *final_h,
                            int32_t *decay_to_end, int32_t *hstate, int B, int L, int C) {
    const int nc = (L + cs - 1) / cs;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int c = 0; c < C; ++c) {
            int32_t s = hstate ? hstate[(int64_t)b * C + c] : 0;
            for (int ci = 0; ci < nc; ++ci) {
                int32_t p = 1 << 30;
                const int t1 = (ci + 1) * cs < L ? (ci + 1) * cs : L;
                for (int t = ci * cs; t < t1; ++t) {
                    int64_t off = ((int64_t)b * L + t) * C + c;
                    s = scan_step(s, n[off], k, u[off]);
                    h[off] = s;
                    p = sat32(floor_shr((int64_t)p * n[off], k));
                }
                int64_t co = ((int64_t)b * nc + ci) * C + c;
                if (final_h) final_h[co] = s;
                if (decay_to_end) decay_to_end[co] = p;
            }
            if (hstate) hstate[(int64_t)b * C + c] = s;
        }
    }
}

/* Chunked multi-head scan (config 4). x[B,L,H,P] i8, Bm/Cm[B,L,H,N] i8,
 * ndec[H] per-head decay numerator, shift k, chunk length cs.
 * y[B,L,H,P] i32; chunk_states[B,nc,H,P,N] (nullable) receives the state at
 * the end of every chunk; hstate[B,H,P,N] nullable in/out.  Follows the
 * chunk loop of ssd_intra_chunk_matmul_kernel (ssd_chunked_scan.py:312-379:
 * per-lane sequential scan inside a chunk, state carried into the next chunk)
 * with the head layout of ssd_multihead (ssd_multihead.py:541-566). */
int mo_ssd_chunked_scan(const int8_t *x, const int8_t *Bm, const int8_t *Cm, const int32_t *ndec,
                        int k, int32_t *y, int32_t *chunk_states, int32_t *hstate, int B, int L,
                        int H, int P, int N, int cs) {
    if (N > 1024 || cs <= 0) return 2;
    int nc = (L + cs - 1) / cs;
#pragma omp parallel for collapse(3) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int hd = 0; hd < H; ++hd) {
            for (int p = 0; p < P; ++p) {
                int32_t h[1024];
                int64_t sbase = (((int64_t)b * H + hd) * P + p) * N;
                for (int n = 0; n < N; ++n) h[n] = hstate ? hstate[sbase + n] : 0;
                int32_t nd = ndec[hd];
                for (int c = 0; c < nc; ++c) {
                    int t0 = c * cs, t1 = t0 + cs < L ? t0 + cs : L;
                    for (int t = t0; t < t1; ++t) {
                        int64_t bth = ((int64_t)b * L + t) * H + hd;
                        int64_t xv = x[bth * P + p];
                        int64_t acc = 0;
                        for (int n = 0; n < N; ++n) {
                            h[n] = scan_step(h[n], nd, k, (int64_t)Bm[bth * N + n] * xv);
                            int64_t term = (int64_t)Cm[bth * N + n] * h[n];
                            if (g_mutation == 3)
                                acc = sat32(acc + term);
                            else
                                acc += term;
                        }
                        y[bth * P + p] = sat32(acc);
                    }
                    if (chunk_states) {
                        int64_t cb = ((((int64_t)b * nc + c) * H + hd) * P + p) * N;
                        for (int n = 0; n < N; ++n) chunk_states[cb + n] = h[n];
                    }
                }
                if (hstate)
                    for (int n = 0; n < N; ++n) hstate[sbase + n] = h[n];
            }
        }
    }
    return 0;
}

/* ------------------------------------------- 2. ternary packing (2 bits) */
static inline uint8_t tern_code(int8_t w) {
    if (g_mutation == 4) return w == 0 ? 0 : (w > 0 ? 3 : 1);
    return w == 0 ? 0 : (w > 0 ? 1 : 3);
}
static inline int8_t tern_decode(unsigned c) {
    /* sign-extend the 2-bit field: 00->0, 01->1, 11->-1, 10->-2 (invalid) */
    return (int8_t)((int)(c << 30) >> 30);
}
/* Position of weight q (0..15) of a 16-weight word: q = 4j + i lives in bits
 * [8i + 2j, 8i + 2j + 1] (spec rule 2). */
static inline int tern_bitpos(int q) { return 8 * (q & 3) + 2 * (q >> 2); }

/* w int8 [N,K] in {-1,0,1} (get_ternary_weights, rational_bitnet.py:215-219)
 * -> packed [N, K/16] little-endian words (= [N, K/4] bytes).  Returns 1 on a
 * value outside {-1,0,1}, 2 when K is not a multiple of 16. */
int mo_pack_ternary(const int8_t *w, uint8_t *p, int N, int K) {
    if (K % 16) return 2;
    int bad = 0;
    for (int64_t n = 0; n < N; ++n)
        for (int wd = 0; wd < K / 16; ++wd) {
            uint32_t word = 0;
            for (int q = 0; q < 16; ++q) {
                int8_t v = w[n * K + 16 * wd + q];
                if (v < -1 || v > 1) bad = 1;
                word |= (uint32_t)tern_code(v) << tern_bitpos(q);
            }
            uint8_t *dst = p + n * (K / 4) + 4 * wd;
            for (int i = 0; i < 4; ++i) dst[i] = (uint8_t)(word >> (8 * i));
        }
    return bad;
}
void mo_unpack_ternary(const uint8_t *p, int8_t *w, int N, int K) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int wd = 0; wd < K / 16; ++wd) {
            const uint8_t *src = p + n * (K / 4) + 4 * wd;
            uint32_t word = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) |
                            ((uint32_t)src[3] << 24);
            for (int q = 0; q < 16; ++q)
                w[n * K + 16 * wd + q] = tern_decode((word >> tern_bitpos(q)) & 3u);
        }
}

/* --------------------------------------------------------- 3. BitLinear */
enum { MO_OUT_INT32 = 0, MO_OUT_INT8 = 1, MO_OUT_DECAY_MOD = 2, MO_OUT_RESIDUAL = 3, MO_OUT_FLOAT = 4 };

__attribute__((target_clones("avx2", "default")))
static int32_t dot_i8(const int8_t *a, const int8_t *w, int K) {
    int32_t s = 0;
    for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)w[k];
    return s;
}

/* a int8 [M,K], wp packed [N,K/4].  Integer accumulate (the exact value of
 * F.linear on integer-valued fp32, rational_bitnet.py:204), then the output
 * kind of spec rule 3.  out: int32/int8/float [M,N] or the int32 residual
 * [M,N] updated in place.  x_scale[M] and w_scale only for MO_OUT_FLOAT. */
void mo_bitlinear_unpacked(const int8_t *a, const int8_t *wu, void *out, int kind, int M, int N, int K, int shift,
                           int32_t res_mult, int res_shift, int32_t res_clamp, const float *x_scale, float w_scale);

void mo_bitlinear(const int8_t *a, const uint8_t *wp, void *out, int kind, int M, int N, int K,
                  int shift, int32_t res_mult, int res_shift, int32_t res_clamp, const float *x_scale,
                  float w_scale) {
    int8_t *wu = (int8_t *)malloc((size_t)N * K);
    mo_unpack_ternary(wp, wu, N, K);
    if (g_mutation == 6) {
        for (int64_t n = 0; n < N; ++n)
            for (int j = 0; j < K / 4; ++j) {
                int8_t *q = wu + n * K + 4 * j, t0 = q[0];
                q[0] = q[3];
                q[3] = t0;
            }
    }
    mo_bitlinear_unpacked(a, wu, out, kind, M, N, K, shift, res_mult, res_shift, res_clamp, x_scale, w_scale);
    free(wu);
}

/* The same with the weights already unpacked to int8 [N][K] (a caller that
 * applies one matrix many times unpacks it once). */
void mo_bitlinear_unpacked(const int8_t *a, const int8_t *wu, void *out, int kind, int M, int N, int K, int shift,
                           int32_t res_mult, int res_shift, int32_t res_clamp, const float *x_scale, float w_scale) {
    /* (row, output) pairs are independent: one flat loop keeps every thread busy
     * at a single row (decode) as well as at many */
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (int m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            int32_t acc = dot_i8(a + (int64_t)m * K, wu + (int64_t)n * K, K);
            int64_t o = (int64_t)m * N + n;
            switch (kind) {
            case MO_OUT_INT32: ((int32_t *)out)[o] = acc; break;
            case MO_OUT_INT8: ((int8_t *)out)[o] = sat8(rshr(acc, shift)); break;
            case MO_OUT_DECAY_MOD: ((int8_t *)out)[o] = (int8_t)clamp64(rshr(acc, shift), -20, 20); break;
            case MO_OUT_RESIDUAL: {
                /* res_clamp > 0: the out_proj output clamp of MambaIntegerBlockV2
                 * (ssd_multihead.py:589-590, spec rule 7.9) on the accumulator */
                int32_t *r = (int32_t *)out;
                int64_t v = res_clamp > 0 ? clamp64(acc, -res_clamp, res_clamp) : acc;
                r[o] = satR((int64_t)r[o] + rshr(v * res_mult, res_shift));
                break;
            }
            case MO_OUT_FLOAT: {
                float sc = w_scale * x_scale[m];
                ((float *)out)[o] = (float)acc * sc;
                break;
            }
            }
        }
    }
}

/* activation_quant_dynamic, 8 bits (rational_bitnet.py:102-111), fp32:
 * scale = max(amax|x|, 1e-8); inv = 127/scale; xq = clamp(rint(x*inv),
 * -127, 127) (rint = round half to even under the default rounding mode, as
 * torch.round); x_scale = scale / 127. */
void mo_act_quant_f32(const float *x, int8_t *xq, float *x_scale, int M, int K) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int m = 0; m < M; ++m) {
        const float *row = x + (int64_t)m * K;
        float amax = 0.0f;
        for (int k = 0; k < K; ++k) {
            float v = fabsf(row[k]);
            amax = v > amax ? v : amax;
        }
        float scale = amax > 1e-8f ? amax : 1e-8f;
        float inv = 127.0f / scale;
        for (int k = 0; k < K; ++k) {
            float q = rintf(row[k] * inv);
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            xq[(int64_t)m * K + k] = (int8_t)q;
        }
        x_scale[m] = scale / 127.0f;
    }
}

/* -------------------------------------------------- 4. integer block ops */
/* BitShiftNorm (mamba_integer_model.py:144-184 table, :200-223, :449-464):
 * spec rule 4.1.  r int32 [T,d] (Q8), gamma int16 [d] (Q8), out int8 [T,d]. */
static void norm_rows(const int32_t *r, const int16_t *gamma, int8_t *out, int T, int d, int kmax, int kmin) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int t = 0; t < T; ++t) {
        const int32_t *row = r + (int64_t)t * d;
        int64_t sum = 0;
        for (int i = 0; i < d; ++i) sum += row[i];
        int64_t mu;
        if (g_mutation == 5)
            mu = sum / d; /* truncation toward zero instead of floor */
        else
            mu = sum >= 0 ? sum / d : -((-sum + d - 1) / d); /* floor */
        int64_t S = 0;
        for (int i = 0; i < d; ++i) {
            int64_t xv = row[i] - mu;
            S += xv * xv;
        }
        int kk = 0;
        for (int j = 1; j <= kmax; ++j)
            if (S >= (int64_t)d << (2 * (j + 8))) kk += 1;
        for (int j = 1; j <= kmin; ++j)
            if (S < (int64_t)d << (2 * (8 - j))) kk -= 1;
        for (int i = 0; i < d; ++i) {
            int64_t xv = row[i] - mu;
            out[(int64_t)t * d + i] = sat8(rshr(xv * gamma[i], 12 + kk));
        }
    }
}

void mo_bitshift_norm(const int32_t *r, const int16_t *gamma, int8_t *out, int T, int d) {
    norm_rows(r, gamma, out, T, d, 8, 3);
}

/* BitShiftNormV2 (ssd_multihead.py:595-632): spec rule 7.1, the V2 table
 * (var >= 4^j -> 2^-j for j <= 6; var < 4^-j -> 2^j for j <= 2). */
void mo_bitshift_norm_v2(const int32_t *r, const int16_t *gamma, int8_t *out, int T, int d) {
    norm_rows(r, gamma, out, T, d, 6, 2);
}

/* Exact squareplus of spec rule 4.4 on the conv output c (Q10) -> int8 Q4. */
int8_t mo_squareplus_q(int32_t c) {
    int64_t v = clamp64(c, -51200, 51200);
    uint64_t s = mo_isqrt((uint64_t)(v * v) + ((uint64_t)1 << 22));
    return sat8(rshr(v + (int64_t)s, 7));
}

/* Depthwise causal conv + squareplus (mamba_integer_model.py:378,404-411;
 * step form conv1d_step.cu:12-58).  xz int8 [B,L,xz_stride] with the x branch
 * in columns [0,D); conv_w int8 [D,4] (Q6), conv_b int32 [D] (Q10);
 * state int8 [B,3,D] (nullable; zeros when null) holds x_{t-3..t-1} before the
 * first position and receives the last three inputs on return.
 * xs int8 [B,L,D]. */
void mo_conv_squareplus(const int8_t *xz, int xz_stride, const int8_t *conv_w,
                        const int32_t *conv_b, int8_t *state, int8_t *xs, int B, int L, int D) {
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d = 0; d < D; ++d) {
            int32_t win[3];
            for (int j = 0; j < 3; ++j) win[j] = state ? state[((int64_t)b * 3 + j) * D + d] : 0;
            for (int t = 0; t < L; ++t) {
                int32_t xv = xz[((int64_t)b * L + t) * xz_stride + d];
                int64_t c = conv_b[d];
                c += (int64_t)conv_w[d * 4 + 0] * win[0];
                c += (int64_t)conv_w[d * 4 + 1] * win[1];
                c += (int64_t)conv_w[d * 4 + 2] * win[2];
                c += (int64_t)conv_w[d * 4 + 3] * xv;
                xs[((int64_t)b * L + t) * D + d] = mo_squareplus_q((int32_t)c);
                win[0] = win[1];
                win[1] = win[2];
                win[2] = xv;
            }
            if (state)
                for (int j = 0; j < 3; ++j) state[((int64_t)b * 3 + j) * D + d] = (int8_t)win[j];
        }
    }
}

/* dt of spec rule 4.8 for dm in [-20, 20] (mamba_integer_model.py:427). */
int32_t mo_dt_q16(int dm) {
    int64_t s = (int64_t)dm * 65536 + (int64_t)mo_isqrt((uint64_t)((int64_t)dm * dm) * ((uint64_t)1 << 32) + ((uint64_t)1 << 34));
    int64_t sq = floor_shr(s, 1);
    return (int32_t)clamp64(rshr(655 * sq, 16), 66, 6554);
}

/* Gate of spec rule 4.11 (mamba_integer_model.py:124-132): Q15 of
 * 0.5 + 0.5 z/(1+|z|) for z in Q4. */
int32_t mo_gate_q15(int z) {
    int64_t a = z < 0 ? -z : z;
    int64_t q = (16384 * a) / (16 + a);
    return (int32_t)(16384 + (z < 0 ? -q : q));
}

/* Fused model scan (spec rules 4.7-4.11; dataflow mamba_integer_model.py:
 * 413-444).  xs int8 [B,L,D]; dm int8 [B,L,D]; xp int8 [B,L,xp_stride] with
 * B at columns [b_off, b_off+N) and C at [b_off+N, b_off+2N); z int8
 * [B,L,z_stride] at column z_off; base int32 [D,N]; k; s_y.
 * yo int8 [B,L,D]; hstate int32 [B,D,N] nullable in/out. */
void mo_block_scan(const int8_t *xs, const int8_t *dm, const int8_t *xp, int xp_stride, int b_off,
                   const int8_t *z, int z_stride, int z_off, const int32_t *base, int k, int s_y,
                   int8_t *yo, int32_t *hstate, int B, int L, int D, int N) {
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d = 0; d < D; ++d) {
            int32_t h[1024];
            for (int n = 0; n < N; ++n) h[n] = hstate ? hstate[((int64_t)b * D + d) * N + n] : 0;
            for (int t = 0; t < L; ++t) {
                int64_t bt = (int64_t)b * L + t;
                int dmv = (int)clamp64(dm[bt * D + d], -20, 20);
                int64_t xd = rshr((int64_t)xs[bt * D + d] * mo_dt_q16(dmv), 10);
                const int8_t *row = xp + bt * xp_stride + b_off;
                int64_t acc = 0;
                for (int n = 0; n < N; ++n) {
                    int32_t nt = (int32_t)clamp64((int64_t)base[(int64_t)d * N + n] + dmv, 0, 32000);
                    h[n] = scan_step(h[n], nt, k, (int64_t)row[n] * xd);
                    acc += (int64_t)row[N + n] * h[n];
                }
                int64_t y = sat32(acc);
                int64_t yg = floor_shr(y * mo_gate_q15(z[bt * z_stride + z_off + d]), 15);
                yo[bt * D + d] = sat8(rshr(yg, s_y));
            }
            if (hstate)
                for (int n = 0; n < N; ++n) hstate[((int64_t)b * D + d) * N + n] = h[n];
        }
    }
}

/* ------------------------------------------ 7. multi-head SSD block (V2) */
/* B / (||B|| + 1e-6) of ssd_multihead.py:552-553 in Q7 (spec rule 7.4):
 * S = sum v^2; nrm = isqrt(S * 2^16); inv = floor(2^30 / nrm);
 * out = sat8(rshr(v * inv, 15)); S = 0 gives zeros. */
void mo_unit_q7(const int8_t *v, int8_t *out, int n) {
    int64_t S = 0;
    for (int i = 0; i < n; ++i) S += (int64_t)v[i] * v[i];
    if (S == 0) {
        for (int i = 0; i < n; ++i) out[i] = 0;
        return;
    }
    int64_t nrm = (int64_t)mo_isqrt((uint64_t)S << 16);
    int64_t inv = ((int64_t)1 << 30) / nrm;
    for (int i = 0; i < n; ++i) out[i] = sat8(rshr((int64_t)v[i] * inv, 15));
}

/* Multi-head SSD scan of MambaIntegerBlockV2 (spec rules 7.3-7.8): the
 * recurrence h_t = exp(A_t) h_{t-1} + B_t (x) X_t, Y_t = C_t . h_t that
 * ssd_multihead_forward (ssd_multihead.py:92-244) evaluates in chunked matmul
 * form, restated sequentially per (b, head, p, n) with the floor rule of
 * dyadic_mamba_kernel.cu:53-56.  xs int8 [B,L,D] (D = H*P); xp int8
 * [B,L,xp_stride] planar: B of head h at [h*N, h*N+N), C at H*N + h*N, dt at
 * 2*H*N + h; z int8 [B,L,z_stride] at column z_off; tab int32 [H][255];
 * yo int8 [B,L,D]; hstate int32 [B,H,P,N] nullable in/out. */
void mo_ssd_v2_scan(const int8_t *xs, const int8_t *xp, int xp_stride, const int8_t *z, int z_stride, int z_off,
                    const int32_t *tab, int s_y, int8_t *yo, int32_t *hstate, int B, int L, int H, int P, int N) {
    const int D = H * P;
    const int64_t ylim = (int64_t)100 << 18;
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int c = 0; c < D; ++c) {
            const int hd = c / P;
            int32_t h[1024];
            int8_t bq[1024], cq[1024];
            for (int n = 0; n < N; ++n) h[n] = hstate ? hstate[((int64_t)b * D + c) * N + n] : 0;
            for (int t = 0; t < L; ++t) {
                const int64_t bt = (int64_t)b * L + t;
                const int8_t *row = xp + bt * xp_stride;
                const int dt = (int)clamp64(row[2 * H * N + hd], -127, 127);
                const int32_t nt = tab[hd * 255 + dt + 127];
                mo_unit_q7(row + hd * N, bq, N);
                mo_unit_q7(row + H * N + hd * N, cq, N);
                const int64_t xv = xs[bt * D + c];
                int64_t acc = 0;
                for (int n = 0; n < N; ++n) {
                    h[n] = scan_step(h[n], nt, 15, (int64_t)bq[n] * xv);
                    acc += (int64_t)cq[n] * h[n];
                }
                const int64_t y = clamp64(sat32(acc), -ylim, ylim);
                const int64_t yg = floor_shr(y * mo_gate_q15(z[bt * z_stride + z_off + c]), 15);
                yo[bt * D + c] = sat8(rshr(yg, s_y));
            }
            if (hstate)
                for (int n = 0; n < N; ++n) hstate[((int64_t)b * D + c) * N + n] = h[n];
        }
    }
}

/* Embedding lookup (mamba_integer_model.py:470,487): r = emb[id] << 4. */
void mo_embed(const int64_t *ids, const int8_t *emb, int32_t *r, int T, int d) {
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < d; ++i) r[(int64_t)t * d + i] = (int32_t)emb[ids[t] * d + i] * 16;
}
