/*
 * mamba_int.h — C ABI of libmamba_int.so, the MI355X (gfx950) integer Mamba
 * inference path (spec mi-spec-2).
 *
 * Conventions (every entry point):
 *   - plain device pointers and sizes; the caller owns every buffer (the
 *     library allocates nothing on the device);
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); all
 *     work is enqueued asynchronously on it, nothing synchronises;
 *   - arguments are validated on the host before anything is enqueued; an
 *     invalid call returns a non-zero mi_status and enqueues nothing;
 *   - mi_last_error_string() describes the last failure of the calling thread;
 *   - a size of zero (batch, len, m, tokens ...) is a valid no-op;
 *   - calls that share no output buffer may run concurrently on different
 *     streams.
 *
 * Reference interfaces replaced (file:line in Jayluci4/mamba-integer):
 *   launch_dyadic_scan           src/cuda_kernels/dyadic_mamba_kernel.cu:135-153
 *   DyadicScanFunction.apply     src/mamba_integer_model.py:260-316
 *   ssd_chunked_scan_forward     src/triton_kernels/ssd_chunked_scan.py:382-422
 *   ssd_multihead_forward        src/triton_kernels/ssd_multihead.py:92-244
 *   BitLinear.forward            src/rational_bitnet.py:167-213
 *   activation_quant_dynamic     src/rational_bitnet.py:88-111
 *   get_ternary_weights          src/rational_bitnet.py:215-219
 *   launch_bitlinear             src/cuda_kernels/bitlinear.cu:18-91
 *   fast_bitnet_matmul           src/triton_kernels/bitnet_kernels.py:198-218
 *   BitShiftNormFunction.forward src/mamba_integer_model.py:200-223
 *   launch_bitshift_norm         src/cuda_kernels/bitshift_norm.cu:9-115
 *   launch_squareplus            src/cuda_kernels/squareplus_kernel.cu:11-68
 *   launch_conv1d_step           src/cuda_kernels/conv1d_step.cu:60-79
 *   MambaIntegerBlock.forward    src/mamba_integer_model.py:396-447
 */
#ifndef MAMBA_INT_H
#define MAMBA_INT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MI_OK = 0,
    MI_ERR_NULL_POINTER = 1,   /* a required pointer is NULL */
    MI_ERR_BAD_DIM = 2,        /* a size is negative, too large or inconsistent */
    MI_ERR_BAD_ALIGNMENT = 3,  /* a pointer or leading dimension breaks the alignment rule */
    MI_ERR_BAD_ARG = 4,        /* a shift, kind or other scalar is out of range */
    MI_ERR_HIP = 5             /* the HIP runtime reported an error at launch */
} mi_status;

/* Output kinds of mi_bitlinear (spec rule 3). */
typedef enum {
    MI_OUT_INT32 = 0,      /* int32 acc */
    MI_OUT_INT8 = 1,       /* int8 sat8(rshr(acc, shift)) */
    MI_OUT_DECAY_MOD = 2,  /* int8 clamp(rshr(acc, shift), -20, 20) */
    MI_OUT_RESIDUAL = 3,   /* int32 r = satR(r + rshr(clamp(acc, +-res_clamp)*res_mult, res_shift)), in place */
    MI_OUT_FLOAT = 4       /* fp32 acc * (w_scale * x_scale[m]) */
} mi_out_kind;

/* Library and spec version, e.g. "libmamba_int 0.2 (mi-spec-2, gfx950)". */
const char *mi_version(void);
/* Message of the calling thread's last failed call ("" if none). */
const char *mi_last_error_string(void);

/* ----------------------------------------------------------------- scans */

/* Dyadic selective scan, config-1 layout (replaces launch_dyadic_scan,
 * dyadic_mamba_kernel.cu:135-153, with the integer rule of :53-59).
 * x int8 [batch,len,d]; b, c int8 [batch,len,nstate]; decay_num int32
 * [d,nstate] in [0, 2^decay_shift]; y int32 [batch,len,d];
 * h_in / h_out int32 [batch,d,nstate], each nullable (NULL h_in = zero state;
 * h_in == h_out allowed).  decay_shift in [1,16]; nstate in [1,128]. */
mi_status mi_dyadic_scan(const int8_t *x, const int8_t *b, const int8_t *c,
                         const int32_t *decay_num, int decay_shift, int32_t *y,
                         const int32_t *h_in, int32_t *h_out, int batch, int len, int d,
                         int nstate, void *stream);

/* Float-compat form with the exact semantics of the reference kernel
 * launch_dyadic_scan (dyadic_mamba_kernel.cu:8-67,134-153): x, h fp32
 * [batch,seq,dim]; nums, shifts int32 [batch,seq,dim] (shift in [0,62]);
 * int64 state; scale_bits in [0,62]. */
mi_status mi_dyadic_scan_f32(const float *x, const int32_t *nums, const int32_t *shifts,
                             float *h, int batch, int seq, int dim, int scale_bits,
                             void *stream);

/* Elementwise recurrence, the integer form of DyadicScanFunction.apply
 * (mamba_integer_model.py:260-316): u, nums int32 [batch,len,channels];
 * h int32 [batch,len,channels] = sat32(floor(h_prev*num / 2^shift) + u);
 * h_in / h_out int32 [batch,channels] nullable.  decay_shift in [1,30].
 * len == 0 with h_out: h_out receives h_in (zeros when h_in is NULL). */
mi_status mi_dyadic_scan_elementwise(const int32_t *u, const int32_t *nums, int decay_shift,
                                     int32_t *h, const int32_t *h_in, int32_t *h_out,
                                     int batch, int len, int channels, void *stream);

/* Chunked elementwise recurrence with the outputs of ssd_chunked_scan_forward
 * (ssd_chunked_scan.py:382-422, chunk loop of :346-379): u, nums int32
 * [batch,len,channels] (per-step decay numerators), one decay_shift (the
 * reference reads shifts[0], :406-409), chunk >= 1.  Outputs:
 *   h            int32 [batch,len,channels]: the state after every step,
 *                sat32(floor(h_prev*num / 2^shift) + u) (the reference's `h`);
 *   final_h      int32 [batch,ceil(len/chunk),channels], nullable: the state at
 *                the last step of each chunk (the reference's `final_h`);
 *   decay_to_end int32 [batch,ceil(len/chunk),channels], nullable: the chunk's
 *                cumulative decay prod(num/2^shift) (the reference's float
 *                `decay_to_end`) in Q30, rounded down after every step:
 *                p = 2^30; p = sat32(floor(p*num / 2^shift)) per step.  With
 *                0 <= num <= 2^shift it lies within len*2^-30 below the exact
 *                product (the floor recurrence has no exact product form).
 * h_in / h_out int32 [batch,channels] nullable (state before / after);
 * len == 0 with h_out: h_out receives h_in (zeros when h_in is NULL). */
mi_status mi_dyadic_chunked_scan(const int32_t *u, const int32_t *nums, int decay_shift, int chunk,
                                 int32_t *h, int32_t *final_h, int32_t *decay_to_end,
                                 const int32_t *h_in, int32_t *h_out, int batch, int len, int channels,
                                 void *stream);

/* Chunked multi-head scan, config-4 layout: the integer form of the SSD scan
 * of ssd_multihead_forward (ssd_multihead.py:92-244: X [B,L,H,P], B/C
 * [B,L,H,N], one decay per head, chunks with the state carried from chunk to
 * chunk, :196-216), with a constant per-head decay numerator.
 * x int8 [batch,len,heads,head_dim]; b, c int8 [batch,len,heads,nstate];
 * decay_num int32 [heads] in [0, 2^decay_shift]; y int32
 * [batch,len,heads,head_dim]; chunk_states int32
 * [batch,ceil(len/chunk),heads,head_dim,nstate] nullable (state at the end of
 * each chunk); h_in / h_out int32 [batch,heads,head_dim,nstate] nullable.
 * Results are identical to the sequential scan for every chunk length. */
mi_status mi_ssd_chunked_scan(const int8_t *x, const int8_t *b, const int8_t *c,
                              const int32_t *decay_num, int decay_shift, int32_t *y,
                              int32_t *chunk_states, const int32_t *h_in, int32_t *h_out,
                              int batch, int len, int heads, int head_dim, int nstate, int chunk,
                              void *stream);

/* ------------------------------------------------------------ BitLinear */

/* Pack ternary int8 [n,k] (values in {-1,0,1}, k % 16 == 0) into the 2-bit
 * layout [n, k/4] (spec rule 2); the storage half of get_ternary_weights
 * (rational_bitnet.py:215-219) and export_int8.py:79-82. */
mi_status mi_pack_ternary(const int8_t *w, uint8_t *packed, int n, int k, void *stream);

/* activation_quant_dynamic, 8 bits (rational_bitnet.py:88-111): x fp32
 * [m,k] -> xq int8 [m,k], x_scale fp32 [m] (= amax/127). */
mi_status mi_act_quant_f32(const float *x, int8_t *xq, float *x_scale, int m, int k,
                           void *stream);

/* out[m, n] = kind(sum_k a[m,k] * W[n,k]) (replaces BitLinear.forward's
 * F.linear + rescale, rational_bitnet.py:204-208, and launch_bitlinear).
 * a int8 [m, lda] (16-byte aligned, lda % 16 == 0); w_packed [n, k/4]
 * (4-byte aligned); out [m, ldo] of the kind's element type (ldo % 4 == 0);
 * k % 16 == 0.  shift in [0,30] for INT8/DECAY_MOD; res_shift in [0,62] and
 * res_clamp >= 0 for RESIDUAL (res_clamp > 0 bounds acc to +-res_clamp before
 * the residual factor: MambaIntegerBlockV2's out clamp to +-100,
 * ssd_multihead.py:589-590; 0 = no bound, MambaIntegerBlock); x_scale [m]
 * and w_scale for FLOAT.  row_stats (RESIDUAL only,
 * nullable, int64 [m,2], 8-byte aligned): the sum and the sum of squares of
 * each updated residual row are added to it with atomics (the caller zeroes
 * it), the row statistics of the next BitShiftNorm.  Chooses the MFMA tile
 * GEMM for m > 64 and the register-unpack GEMV path for m <= 64. */
mi_status mi_bitlinear(const int8_t *a, int lda, const uint8_t *w_packed, void *out, int ldo,
                       int kind, int m, int n, int k, int shift, int32_t res_mult, int res_shift,
                       int32_t res_clamp, const float *x_scale, float w_scale, int64_t *row_stats,
                       void *stream);
/* Same contract, forcing the MFMA tile GEMM (prefill path). */
mi_status mi_bitlinear_gemm(const int8_t *a, int lda, const uint8_t *w_packed, void *out,
                            int ldo, int kind, int m, int n, int k, int shift, int32_t res_mult,
                            int res_shift, int32_t res_clamp, const float *x_scale, float w_scale,
                            int64_t *row_stats, void *stream);
/* Same contract, forcing the decode GEMV (m <= 64). */
mi_status mi_bitlinear_gemv(const int8_t *a, int lda, const uint8_t *w_packed, void *out,
                            int ldo, int kind, int m, int n, int k, int shift, int32_t res_mult,
                            int res_shift, int32_t res_clamp, const float *x_scale, float w_scale,
                            int64_t *row_stats, void *stream);
/* The decode out_proj with the next norm's row statistics as per-block
 * partials instead of atomics (the residual update of BitLinear.forward +
 * MambaIntegerBlock.forward's residual add, mamba_integer_model.py:446-447,
 * for m <= 64 tokens): r[m, n] (int32, row stride ldr) is updated as by
 * mi_bitlinear_gemv RESIDUAL (res_clamp as there), and stats_parts int64 [m, ceil(n/16), 2]
 * receives, for every row i and block b of 16 features, the sum and the sum
 * of squares of the updated r[i, 16b : 16b+16] (plain stores: no zeroing,
 * no atomics).  The norm entries below sum them (their stats_parts =
 * ceil(n/16)).  m <= 64; k % 64 == 0; a, w_packed, stats_parts 16-byte
 * aligned. */
mi_status mi_bitlinear_residual_parts(const int8_t *a, int lda, const uint8_t *w_packed, int32_t *r,
                                      int ldr, int m, int n, int k, int32_t res_mult, int res_shift,
                                      int32_t res_clamp, int64_t *stats_parts, void *stream);

/* ---------------------------------------------------------- block ops */

/* Integer BitShiftNorm (spec rule 4.1; mamba_integer_model.py:144-184,
 * 200-223): r int32 [tokens,dim] (Q8) -> out int8 [tokens,dim]; gamma int16
 * [dim] (Q8). dim in [1, 8192].  row_stats (nullable, int64 [tokens,2] =
 * (sum r, sum r^2) per row, as mi_embed / RESIDUAL outputs accumulate them)
 * turns the norm into an elementwise pass (dim % 4 == 0, r 16-byte aligned). */
mi_status mi_bitshift_norm(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens,
                           int dim, const int64_t *row_stats, void *stream);

/* mi_bitshift_norm (v2 != 0: mi_bitshift_norm_v2) with the row statistics
 * given as per-block partials: stats_parts int64 [tokens, nparts, 2] (16-byte
 * aligned), the (sum, sum of squares) pairs that mi_bitlinear_residual_parts
 * stores per 16 output features, summed per row here.  dim % 4 == 0, r
 * 16-byte aligned.  For batches whose norm would otherwise reduce its rows. */
mi_status mi_bitshift_norm_parts(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens, int dim,
                                 const int64_t *stats_parts, int nparts, int v2, void *stream);

/* Embedding (mamba_integer_model.py:470,487): r[t,:] = emb[ids[t],:] << 4.
 * ids int64 [tokens] (an id outside [0,vocab) gives a zero row), emb int8
 * [vocab,dim], r int32.  row_stats (nullable, int64
 * [stats_layers,tokens,2]): layer 0 receives the row statistics of r, layers
 * 1..stats_layers-1 are zeroed for the residual epilogues that follow. */
mi_status mi_embed(const int64_t *ids, const int8_t *emb, int32_t *r, int tokens, int dim,
                   int vocab, int64_t *row_stats, int stats_layers, void *stream);

/* Depthwise causal conv (width 4) + squareplus (spec rules 4.3-4.4;
 * mamba_integer_model.py:378,404-411; step form conv1d_step.cu:12-58).
 * xz int8 [batch,len,xz_stride], x branch in columns [0,d_inner);
 * conv_w int8 [d_inner,4]; conv_b int32 [d_inner]; state_in / state_out int8
 * [batch,3,d_inner] nullable (NULL state_in = zeros; in == out allowed);
 * xs int8 [batch,len,d_inner]. */
mi_status mi_conv_squareplus(const int8_t *xz, int xz_stride, const int8_t *conv_w,
                             const int32_t *conv_b, const int8_t *state_in, int8_t *state_out,
                             int8_t *xs, int batch, int len, int d_inner, void *stream);

/* Prefill in_proj with the conv + squareplus of its x half fused into the
 * GEMM epilogue: in_proj, chunk, conv1d, clamp and squareplus of
 * MambaIntegerBlock.forward (mamba_integer_model.py:400-411), the steps the
 * reference fuses as fused_squareplus_clamp (fused_activations.py:89-119,
 * 229-262).  a int8 [batch*len, lda] (the normalized rows), w_in packed
 * [2*d_inner, d_model/16 words] (16-byte aligned), shift = in_proj requant
 * shift.  Writes xs int8 [batch*len, d_inner] = squareplus(conv(x)), the z
 * half into xz columns [d_inner, 2*d_inner) (row stride ldxz, 16-byte
 * aligned; the x half is not written) and state_out [batch,3,d_inner] = the
 * last three x rows of each sequence; state_in [batch,3,d_inner] nullable
 * (zeros), and must not overlap state_out.  Identical to mi_bitlinear
 * (MI_OUT_INT8) followed by mi_conv_squareplus.  d_inner % 128 == 0,
 * d_model % 64 == 0.  len == 0: only state_out is written, = state_in
 * (zeros when state_in is NULL). */
mi_status mi_in_proj_conv(const int8_t *a, int lda, const uint8_t *w_in, int shift,
                          const int8_t *conv_w, const int32_t *conv_b, const int8_t *state_in,
                          int8_t *state_out, int8_t *xs, int8_t *xz, int ldxz, int batch, int len,
                          int d_model, int d_inner, void *stream);

/* Fused model scan (spec rules 4.7-4.11; MambaIntegerBlock.forward,
 * mamba_integer_model.py:413-444): decay from base + dm, dt from dm, input
 * xs*dt (x) B, scan, y = C.h, gate by z, requant.
 * xs, dm int8 [batch,len,d_inner]; xp int8 [batch,len,xp_stride] with B at
 * columns [b_off, b_off+nstate) and C at [b_off+nstate, b_off+2*nstate);
 * z int8 [batch,len,z_stride] at column z_off; base int32 [d_inner,nstate] in
 * [0,32000]; yo int8 [batch,len,d_inner]; h_in / h_out int32
 * [batch,d_inner,nstate] nullable.  decay_shift == 15; nstate in [1,64];
 * s_y in [0,30]. */
mi_status mi_block_scan(const int8_t *xs, const int8_t *dm, const int8_t *xp, int xp_stride,
                        int b_off, const int8_t *z, int z_stride, int z_off,
                        const int32_t *base, int decay_shift, int s_y, int8_t *yo,
                        const int32_t *h_in, int32_t *h_out, int batch, int len, int d_inner,
                        int nstate, void *stream);

/* BitShiftNormV2 (ssd_multihead.py:595-632; spec rule 7.1): mi_bitshift_norm
 * with the V2 threshold table (scales 2^-1 .. 2^-6 for var >= 4 .. 4096, 2
 * and 4 for var < 1/4 and < 1/16), the norm of the multi-head SSD block. */
mi_status mi_bitshift_norm_v2(const int32_t *r, const int16_t *gamma, int8_t *out, int tokens,
                              int dim, const int64_t *row_stats, void *stream);

/* Scan of the multi-head SSD block (MambaIntegerBlockV2.forward,
 * ssd_multihead.py:536-586, over ssd_multihead_forward :92-244; spec rules
 * 7.3-7.8): per token and head, B and C scaled to unit vectors (Q7), the
 * decay decay_tab[h][dt + 127] (int32 [n_heads][255] in [0, 32768], shift
 * 15), h = floor(h * n / 2^15) + B (x) x, y = C . h clamped to +-100 (Q18),
 * gate by z, requant by s_y.  xs int8 [batch,len,d_inner] (d_inner =
 * n_heads * d_head, d_head % 16 == 0); xp int8 [batch,len,xp_stride] planar:
 * B of head h at columns [h*nstate, (h+1)*nstate), C at n_heads*nstate +
 * h*nstate, dt at 2*n_heads*nstate + h; z int8 [batch,len,z_stride] at
 * column z_off; yo int8 [batch,len,d_inner]; h_in / h_out int32
 * [batch,n_heads,d_head,nstate] nullable (in == out allowed).  nstate in
 * {16, 32, 64}; rows and xs/xp/z/yo 16-byte aligned. */
mi_status mi_ssd_block_scan(const int8_t *xs, const int8_t *xp, int xp_stride, const int8_t *z,
                            int z_stride, int z_off, const int32_t *decay_tab, int n_heads, int s_y,
                            int8_t *yo, const int32_t *h_in, int32_t *h_out, int batch, int len,
                            int d_inner, int nstate, void *stream);

/* Greedy pick (scripts/sft_mamba_integer.py:138-141 argmax): out[r] = first
 * index of the maximum of logits[r, 0:cols] (int32 [rows, ld]). */
mi_status mi_argmax_i32(const int32_t *logits, int ld, int64_t *out, int rows, int cols,
                        void *stream);

/* ------------------------------------------------ fused decode stages */
/* A decode step at small batch is bound by its chain of dependent kernels;
 * these entries fuse the per-token stages of MambaIntegerBlock.forward
 * (mamba_integer_model.py:396-447) and the one-step conv of
 * launch_conv1d_step (conv1d_step.cu:60-79).  Same integer rules as the
 * unfused ops, bit for bit.
 *
 * Row statistics of the norm entries: row_stats NULL (each block reduces
 * the rows itself) or int64 [m, stats_parts, 2], row i's (sum r, sum r^2)
 * being the sum over its parts: stats_parts = 1 for the full sums of
 * mi_embed / RESIDUAL atomics (8-byte aligned), ceil(d/16) for the partials
 * of mi_bitlinear_residual_parts (16-byte aligned); stats_parts <= 4096. */

/* BitShiftNorm of r (int32 [m,k], m <= 64 (16-token row groups, one block
 * row each), k % 64 == 0, k <= 3072; r and
 * w_packed 16-byte, gamma 8-byte aligned) fused into
 * the BitLinear GEMV: out[m, n] = INT8 (sat8(rshr(acc, shift))) or INT32 acc,
 * out row stride ldo.  Replaces BitShiftNorm.forward + BitLinear.forward for
 * one token per sequence (the lm_head path of MambaIntegerModel.forward,
 * mamba_integer_model.py:492-494). */
mi_status mi_norm_bitlinear(const int32_t *r, const int64_t *row_stats, int stats_parts,
                            const int16_t *gamma, const uint8_t *w_packed, void *out, int ldo, int kind,
                            int m, int n, int k, int shift, void *stream);

/* Norm + in_proj (INT8, shift s_in) + depthwise conv step + squareplus:
 * r int32 [m,d_model]; w_in packed [2*d_inner, d_model/4]; the x half goes
 * through the conv with conv_state int8 [m,3,d_inner] updated in place and
 * lands in xs int8 [m,d_inner]; the z half is written to xz int8
 * [m,2*d_inner] at columns [d_inner, 2*d_inner).  m <= 64, d_model <= 3072;
 * alignment as mi_norm_bitlinear. */
mi_status mi_norm_in_proj_conv(const int32_t *r, const int64_t *row_stats, int stats_parts,
                               const int16_t *gamma, const uint8_t *w_in, int s_in,
                               const int8_t *conv_w, const int32_t *conv_b, int8_t *conv_state,
                               int8_t *xs, int8_t *xz, int m, int d_model, int d_inner, void *stream);

/* mi_norm_in_proj_conv with BitShiftNormV2's threshold table (spec rule
 * 7.1): the first decode stage of the multi-head SSD block
 * (MambaIntegerBlockV2.forward, ssd_multihead.py:523-536). */
mi_status mi_norm_v2_in_proj_conv(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                  const int16_t *gamma, const uint8_t *w_in, int s_in,
                                  const int8_t *conv_w, const int32_t *conv_b, int8_t *conv_state,
                                  int8_t *xs, int8_t *xz, int m, int d_model, int d_inner, void *stream);

/* dt_proj (DECAY_MOD, shift s_dt) + decay + dt + one scan step + y + gate +
 * requant (spec rules 4.6-4.11 at L = 1): xp int8 [m,xp_stride] (dt_raw at
 * [0,dt_rank), B, C after it); w_dt packed [d_inner, dt_rank/4]; xs int8
 * [m,d_inner]; z int8 [m,z_stride] at column z_off; base int32
 * [d_inner,nstate]; h_state int32 [m,d_inner,nstate] updated in place;
 * yo int8 [m,d_inner].  dt_rank % 16 == 0, <= 256; nstate <= 64; m <= 65535
 * (also for mi_xpart_dt_scan_step, mi_xproj_dt_scan_step, mi_conv_step_xpart). */
mi_status mi_dt_scan_step(const int8_t *xp, int xp_stride, int dt_rank, const uint8_t *w_dt, int s_dt,
                          const int8_t *xs, const int8_t *z, int z_stride, int z_off, const int32_t *base,
                          int decay_shift, int s_y, int32_t *h_state, int8_t *yo, int m, int d_inner,
                          int nstate, void *stream);

/* x_proj (INT8, shift s_x) fused in front of mi_dt_scan_step: each block
 * computes the dt_rank + 2*nstate x_proj outputs of its token from xs int8
 * [m,d_inner] (16-byte aligned) and w_x packed [dt_rank+2*nstate,
 * d_inner/4] (8-byte aligned), then runs the dt_proj + scan step + gate of
 * mi_dt_scan_step.  dt_rank + 2*nstate <= 256; d_inner % 32 == 0. */
mi_status mi_xproj_dt_scan_step(const int8_t *xs, const uint8_t *w_x, int s_x, int dt_rank,
                                const uint8_t *w_dt, int s_dt, const int8_t *z, int z_stride, int z_off,
                                const int32_t *base, int decay_shift, int s_y, int32_t *h_state,
                                int8_t *yo, int m, int d_inner, int nstate, void *stream);

/* mi_norm_in_proj_conv that also starts x_proj (self.x_proj,
 * mamba_integer_model.py:379,414): the block owning channels [16b, 16b+16)
 * of the x half writes the exact int32 partial
 *   xpart[i, b, n] = sum over those channels c of w_x[n, c] * xs[i, c]
 * into xpart int32 [m, d_inner/16, nx], w_x packed [nx, d_inner/4]
 * (4-byte aligned), nx = dt_rank + 2*nstate <= 256. */
mi_status mi_norm_in_proj_conv_xpart(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                     const int16_t *gamma, const uint8_t *w_in, int s_in,
                                     const int8_t *conv_w, const int32_t *conv_b,
                                     int8_t *conv_state, int8_t *xs, int8_t *xz, const uint8_t *w_x, int nx,
                                     int32_t *xpart, int m, int d_model, int d_inner, void *stream);

/* The decode conv step followed by x_proj, for widths where the in_proj
 * stage does not carry the conv (conv1d_step.cu:12-58, then self.x_proj,
 * mamba_integer_model.py:378-379,404-414): one token per sequence, the x half
 * of xz int8 [m, xz_stride] (columns 0..d_inner-1) through the depthwise conv
 * step + squareplus with conv_state int8 [m,3,d_inner] shifted in place ->
 * xs int8 [m,d_inner], then xp int8 [m, xp_stride] = sat8(rshr(xs @ w_x^T,
 * s_x)) for w_x packed [nx, d_inner/4], nx <= 256.  w_x, conv_w int8
 * [d_inner,4] and conv_b int32 [d_inner] 16-byte aligned.  One block per
 * token; d_inner a multiple of 256, <= 8192.  The row feeds mi_dt_scan_step. */
mi_status mi_conv_step_xproj(const int8_t *xz, int xz_stride, const int8_t *conv_w, const int32_t *conv_b,
                             int8_t *conv_state, int8_t *xs, const uint8_t *w_x, int s_x, int nx, int8_t *xp,
                             int xp_stride, int m, int d_inner, void *stream);

/* mi_conv_step_xproj with x_proj left as exact int32 partial sums over the
 * four channel quarters (same reference lines):
 *   xpart[i, q, n] = sum over c in [q*d_inner/4, (q+1)*d_inner/4) of
 *                    w_x[n, c] * xs[i, c]
 * into xpart int32 [m, 4, nx]; xs and conv_state as in mi_conv_step_xproj.
 * Four blocks per token share its conv operands and x_proj weights.
 * d_inner a multiple of 1024, <= 8192; nx <= 256.  The partials feed
 * mi_xpart_dt_scan_step with nblk = 4.  (No reference counterpart of the
 * split; it replaces the same conv1d_step.cu + x_proj pair.) */
mi_status mi_conv_step_xpart(const int8_t *xz, int xz_stride, const int8_t *conv_w, const int32_t *conv_b,
                             int8_t *conv_state, int8_t *xs, const uint8_t *w_x, int nx, int32_t *xpart, int m,
                             int d_inner, void *stream);

/* mi_dt_scan_step with x_proj finished from those partials:
 * xp[i, n] = sat8(rshr(sum over b < nblk of xpart[i, b, n], s_x)), then
 * dt_rank, B and C as in mi_dt_scan_step.  nblk = d_inner/16 for the
 * partials of mi_norm_in_proj_conv_xpart, 4 for mi_conv_step_xpart. */
mi_status mi_xpart_dt_scan_step(const int32_t *xpart, int nblk, int s_x, int dt_rank, const uint8_t *w_dt,
                                int s_dt, const int8_t *xs, const int8_t *z, int z_stride, int z_off,
                                const int32_t *base, int decay_shift, int s_y, int32_t *h_state, int8_t *yo,
                                int m, int d_inner, int nstate, void *stream);

/* ------------------------------------------------ greedy pick */
/* The generation loop's argmax (scripts/inference.py:147-161, torch.argmax
 * over the last logits) fused into the lm_head: mi_norm_bitlinear (INT32)
 * in 64-output blocks, each block also writing for every row i its partial
 * key keys[i, b] = max over its outputs j of (logit << 32 | 0x7FFFFFFF - j),
 * so the largest key of a row names its first maximal index.  keys int64
 * [m, ceil(n/64)]; logits int32 [m, ldo] or NULL (then not stored). */
mi_status mi_norm_bitlinear_argmax(const int32_t *r, const int64_t *row_stats, int stats_parts,
                                   const int16_t *gamma, const uint8_t *w_packed, int32_t *logits, int ldo,
                                   int64_t *keys, int m, int n, int k, void *stream);

/* ids[i] = the index the largest of keys[i, 0:nkeys] names (int64 out). */
mi_status mi_argmax_keys(const int64_t *keys, int nkeys, int64_t *ids, int rows, void *stream);

/* mi_argmax_keys, then mi_embed (with row statistics) of the picked ids;
 * the ids are written to ids. */
mi_status mi_embed_argmax(const int64_t *keys, int nkeys, int64_t *ids, const int8_t *emb, int32_t *r,
                          int tokens, int dim, int vocab, int64_t *row_stats, int stats_layers, void *stream);

/* ------------------------------------------------ whole decode step */
/* Integer parameters of one layer (device pointers; spec mi-spec-2 layouts:
 * packed ternary matrices [rows][cols/4] bytes, 16-byte aligned).  The
 * dyadic-scan block uses w_dt, s_dt and base; the multi-head SSD block
 * (MI_BLOCK_SSD) w_x with the planar rows of spec rule 7.3 and decay_tab. */
typedef struct mi_layer_params {
    const int16_t *gamma;    /* BitShiftNorm gain [d_model] */
    const uint8_t *w_in;     /* in_proj [2*d_inner][d_model/4] */
    int s_in;                /* in_proj requant shift */
    const int8_t *conv_w;    /* [d_inner][4] taps */
    const int32_t *conv_b;   /* [d_inner] */
    const uint8_t *w_x;      /* x_proj [dt_rank+2*d_state][d_inner/4] */
    int s_x;
    const uint8_t *w_dt;     /* dt_proj [d_inner][dt_rank/4] */
    int s_dt;
    const int32_t *base;     /* decays [d_inner][d_state] */
    int decay_shift;
    int s_y;
    const uint8_t *w_out;    /* out_proj [d_model][d_inner/4] */
    int32_t res_mult;
    int res_shift;
    const int32_t *decay_tab; /* SSD block: [n_heads][255] decay numerators */
    int32_t out_clamp;        /* out_proj accumulator bound, the res_clamp of
                                 mi_bitlinear RESIDUAL (SSD block: spec rule 7.9;
                                 0 = none, the dyadic block) */
} mi_layer_params;

enum { MI_BLOCK_DYADIC = 0, MI_BLOCK_SSD = 1 };

/* The model: dims, int8 embedding [vocab][d_model], `layers` a HOST array of
 * n_layer entries, final gain and packed lm_head [vocab][d_model/4].  block
 * MI_BLOCK_DYADIC: d_inner = 2*d_model (MambaIntegerBlock); MI_BLOCK_SSD:
 * d_inner = n_heads*d_head (MambaIntegerBlockV2, dt_rank unused). */
typedef struct mi_model_params {
    int d_model, n_layer, vocab_size, d_state, dt_rank;
    const int8_t *emb;
    const mi_layer_params *layers;
    const int16_t *gamma_f;
    const uint8_t *w_head;
    int block, n_heads, d_head;
} mi_model_params;

/* Bytes of the caller-owned device workspace mi_decode_step needs at batch m
 * (1 <= m <= 64; d_model % 64 == 0, <= 3072; dyadic block: dt_rank % 16 ==
 * 0 and dt_rank + 2*d_state <= 256; SSD block: d_head % 16 == 0, d_state in
 * {16, 32, 64}). */
mi_status mi_decode_workspace_size(const mi_model_params *params, int m, size_t *bytes);

/* One greedy decode step of the whole model for m sequences (the reference's
 * generation step, scripts/inference.py:147-161 over MambaIntegerModel.forward,
 * mamba_integer_model.py:486-495, with recurrent state; the dyadic block runs
 * the three fused stages per layer for d_model <= 1024 and m * d_model^2 <=
 * 64 * 768^2, otherwise five batched stages (norm from statistics partials,
 * in_proj GEMV, mi_conv_step_xproj, mi_dt_scan_step, out_proj) where
 * d_inner % 256 == 0; the SSD block four): ids int64 [m] in, next_ids int64
 * [m] out (first maximal logit), logits int32 [m][ld_logits] when non-NULL;
 * conv_state / h_state are HOST arrays of n_layer device pointers (int8
 * [m][3][d_inner], int32 [m][d_inner][d_state]) updated in place; workspace
 * 256-byte aligned, at least mi_decode_workspace_size bytes (which depends on
 * the path).  Enqueues only kernels and device copies (no allocation, no
 * memset): graph-capturable. */
mi_status mi_decode_step(const mi_model_params *params, int m, const int64_t *ids, int64_t *next_ids,
                         int32_t *logits, int ld_logits, int8_t *const *conv_state, int32_t *const *h_state,
                         void *workspace, size_t workspace_bytes, void *stream);

/* mi_decode_step for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It has no counterpart in the reference.  The workspace is a file-scope
 * device array of the library, 16 MiB (16777216 bytes) per GPU: every process
 * that runs any kernel of this library on a GPU holds it there until the
 * process ends, whether or not it calls this entry.  Its address (and an
 * event) are set up once per device on the first call, with that device
 * current; make that first call outside stream capture.  A model and batch
 * whose workspace (mi_decode_workspace_size) exceeds 16 MiB is rejected with
 * MI_ERR_BAD_DIM before anything is enqueued; the d768 x 24 model fits up to
 * m = 64 and the d2048 x 48 model (batched stages, vocab 32000) up to m = 64.
 * Every call on one GPU shares that array, so calls must not overlap on one
 * GPU: a call on another stream than the previous eager call, while that one
 * is still running, is refused with MI_ERR_BAD_ARG; calls from several host
 * threads are serialized.  Replays of a captured step are not tracked: the
 * caller orders them against other calls.  The step writes every part of the
 * workspace it reads, so nothing needs clearing between calls.  Same
 * arguments and results as mi_decode_step otherwise. */
mi_status mi_decode_step_static(const mi_model_params *params, int m, const int64_t *ids, int64_t *next_ids,
                                int32_t *logits, int ld_logits, int8_t *const *conv_state,
                                int32_t *const *h_state, void *stream);

/* ------------------------------------------------ integer checkpoints */
/* The integer parameters above in a versioned file (format 2, spec
 * mi-spec-2; format-1 files of mi-spec-1, whose SSD layers have no out_proj
 * clamp, are read as well): a 128-byte header (magic "MIQCKPT", format, spec string, dims,
 * logit_scale, table CRC, block type and heads), a table of named
 * little-endian tensors (dtype,
 * shape, offset, bytes, CRC-32), and the tensors at 256-byte aligned offsets:
 * 2-bit packed ternary matrices, int8 embedding and conv taps, int32 conv
 * bias and decay numerators, int16 gains, and the per-layer shifts.
 * Replaces the reference's inference export (scripts/export_int8.py:50-135,
 * magic 0xDAD1C: float embedding, conv and gains, one byte per ternary
 * weight plus a float scale) and its loader load_model
 * (src/cpp_engine/mamba_infer.cpp:46-118), which exit()s on any error and
 * allocates every tensor itself.  Files are written by
 * mamba_int.checkpoint.save and converted from the reference's float state
 * dicts by mamba_int.checkpoint.convert_state_dict. */
typedef struct mi_checkpoint mi_checkpoint;

typedef struct mi_checkpoint_info {
    int format_version;
    char spec[16];             /* "mi-spec-2" (format 2) or "mi-spec-1" (format 1) */
    int d_model, n_layer, vocab_size, d_state, dt_rank;
    float logit_scale;         /* float logits = int32 logits * logit_scale (> 0) */
    size_t device_bytes;       /* bytes mi_checkpoint_upload fills */
    int block, n_heads, d_head; /* MI_BLOCK_DYADIC or MI_BLOCK_SSD (then n_heads, d_head) */
} mi_checkpoint_info;

/* Reads a checkpoint into host memory and validates it: magic, format,
 * spec, dims, table CRC, every tensor's dtype, shape (against the dims),
 * alignment and CRC-32, the ternary codes, the shifts (decay shift 15),
 * decays in [0, 32000] and the out_proj clamps (>= 1 in format-2 SSD layers,
 * 0 elsewhere).  *out is NULL on failure; close with
 * mi_checkpoint_close. */
mi_status mi_checkpoint_open(const char *path, mi_checkpoint **out);
mi_status mi_checkpoint_get_info(const mi_checkpoint *ck, mi_checkpoint_info *info);
/* Copies every tensor into `device` (256-byte aligned, at least
 * info.device_bytes) on `stream`, waits for the copies, and fills *params
 * (its `layers` = the caller's HOST array `layers` of n_layers = n_layer
 * entries) with pointers into `device`, ready for mi_decode_step.  No device
 * allocation. */
mi_status mi_checkpoint_upload(const mi_checkpoint *ck, void *device, size_t device_bytes,
                               mi_model_params *params, mi_layer_params *layers, int n_layers,
                               void *stream);
void mi_checkpoint_close(mi_checkpoint *ck);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_INT_H */
