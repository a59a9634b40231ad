// One greedy decode step of the whole model behind the C ABI (host-side
// orchestration of the fused decode stages; no device allocation, no memset,
// so a caller may capture it in a HIP graph).
//
// Per step: embed the input ids (with their row statistics), then for every
// layer the three fused stages (norm + in_proj + conv + x_proj partials;
// x_proj finish + dt_proj + scan step + gate; out_proj + residual + per-block
// row-statistics partials, which the next norm sums), then norm + lm_head
// with the greedy pick fused in, and the pick itself.  Wide models and large
// batches (where every fused block would normalize m rows of d_model) run the
// batched stages instead: norm from the partials, in_proj GEMV, conv step +
// x_proj, dt_proj + scan step, out_proj with partials; the head as norm,
// GEMV and argmax.  Mirrors the reference's
// generation step (scripts/inference.py:147-161 over
// MambaIntegerModel.forward, src/mamba_integer_model.py:486-495) with the
// recurrent state of a Mamba decode instead of a full-prefix recompute.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "mi_common.hpp"

namespace mi {
namespace {

constexpr size_t kAlign = 256;
size_t up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct WsLayout {
    size_t r, stats, parts, xz, xs, xp, yo, xpart, keys, a, logits, xq, total;
};

bool ssd(const mi_model_params &p) { return p.block == MI_BLOCK_SSD; }
size_t d_inner(const mi_model_params &p) { return ssd(p) ? (size_t)p.n_heads * p.d_head : 2 * (size_t)p.d_model; }
// x_proj width of the SSD block: planar B, C, dt rounded up to 16 (spec rule 7.3)
size_t ssd_xp_width(const mi_model_params &p) {
    return ((size_t)2 * p.n_heads * p.d_state + p.n_heads + 15) / 16 * 16;
}

// x_proj row width of the dyadic block's batched stages (dt_rank + 2*nstate, to 16)
size_t dyadic_xp_width(const mi_model_params &p) { return ((size_t)p.dt_rank + 2 * p.d_state + 15) / 16 * 16; }

// The dyadic block's fused stages normalize all m rows in every block, so the
// repeated work grows as m * d^2: the same rule as the Python runner (fused for
// d_model <= 1024 and m * d^2 <= 64 * 768^2), the batched stages otherwise,
// where their limits allow (d_inner a multiple of 256 up to 8192).
bool batched(const mi_model_params &p, int m) {
    if (ssd(p)) return false;
    const int64_t d = p.d_model, D = (int64_t)d_inner(p);
    const bool fused_ok = d <= 1024 && m * d * d <= 64 * 768 * 768;
    return !fused_ok && D % 256 == 0 && D <= 8192 && p.dt_rank + 2 * p.d_state <= 256;
}

// The batched stages' conv step leaves x_proj as int32 sums over four channel
// quarters (mi_conv_step_xpart) where d_inner is a multiple of 1024.
bool quarters(const mi_model_params &p) { return d_inner(p) % 1024 == 0; }

// Sub-buffer offsets of the decode workspace for batch m.
WsLayout ws_layout(const mi_model_params &p, int m) {
    const size_t d = p.d_model, D = d_inner(p), N = p.d_state, R = p.dt_rank, V = p.vocab_size;
    WsLayout w{};
    size_t o = 0;
    w.r = o; o += up((size_t)m * d * 4);
    w.stats = o; o += up((size_t)m * 2 * 8);
    w.keys = o; o += up((size_t)m * ((V + 63) / 64) * 8);
    w.xz = o; o += up((size_t)m * 2 * D);
    w.xs = o; o += up((size_t)m * D);
    w.yo = o; o += up((size_t)m * D);
    w.parts = o; o += up((size_t)m * (d / 16) * 2 * 8);
    if (ssd(p)) {
        w.xp = o; o += up((size_t)m * ssd_xp_width(p));
    } else if (batched(p, m)) {
        w.xp = o; o += up((size_t)m * dyadic_xp_width(p));
        w.a = o; o += up((size_t)m * d);
        w.logits = o; o += up((size_t)m * ((V + 3) / 4 * 4) * 4);
        if (quarters(p)) {
            w.xq = o; o += up((size_t)m * 4 * (R + 2 * N) * 4);
        }
    } else {
        w.xpart = o; o += up((size_t)m * (D / 16) * (R + 2 * N) * 4);
    }
    w.total = o;
    return w;
}

mi_status check_model(const char *fn, const mi_model_params *p, int m) {
    MI_REQUIRE(p, MI_ERR_NULL_POINTER, "%s: params is NULL", fn);
    MI_REQUIRE(m >= 1 && m <= 64, MI_ERR_BAD_DIM, "%s: m=%d outside [1,64] (the fused decode stages)", fn, m);
    MI_REQUIRE(p->n_layer >= 1 && p->vocab_size >= 1, MI_ERR_BAD_DIM, "%s: n_layer and vocab_size must be >= 1", fn);
    MI_REQUIRE(p->d_model >= 64 && p->d_model % 64 == 0 && p->d_model <= 3072, MI_ERR_BAD_DIM,
               "%s: d_model=%d must be a multiple of 64 in [64,3072]", fn, p->d_model);
    MI_REQUIRE(p->block == MI_BLOCK_DYADIC || p->block == MI_BLOCK_SSD, MI_ERR_BAD_ARG, "%s: block=%d unknown", fn,
               p->block);
    if (ssd(*p)) {
        MI_REQUIRE(p->n_heads >= 1 && p->d_head >= 16 && p->d_head % 16 == 0 &&
                       (p->d_state == 16 || p->d_state == 32 || p->d_state == 64),
                   MI_ERR_BAD_DIM, "%s: n_heads=%d, d_head=%d, d_state=%d outside the SSD block's limits", fn,
                   p->n_heads, p->d_head, p->d_state);
    } else {
        MI_REQUIRE(p->dt_rank >= 16 && p->dt_rank % 16 == 0 && p->d_state >= 1 && p->d_state <= 64 &&
                       p->dt_rank + 2 * p->d_state <= 256,
                   MI_ERR_BAD_DIM, "%s: dt_rank=%d, d_state=%d outside the fused stages' limits", fn, p->dt_rank,
                   p->d_state);
    }
    MI_REQUIRE(p->emb && p->layers && p->gamma_f && p->w_head, MI_ERR_NULL_POINTER,
               "%s: emb, layers, gamma_f and w_head are required", fn);
    return MI_OK;
}

// The workspace of mi_decode_step_static: one array in device memory per GPU,
// reserved wherever the library's code object is loaded on a GPU (its first
// kernel launch there) and held until the process ends, whether or not the
// static entry is called (no allocation call).  Host code never uses the name
// `scratch` as an address (on the host it is a stand-in symbol); it uses the
// per-device address hipGetSymbolAddress returns.
//
// Calls share the array, so two calls whose kernels overlap on one GPU would
// race.  Each device keeps the stream of its last eager call and an event
// recorded after it: a call on another stream while that event is pending is
// refused.  Host threads are serialized by one mutex, so check and record are
// one step.  Work under stream capture is neither checked nor recorded (the
// graph's replays are the caller's to order).
constexpr size_t kStaticScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
struct StaticSlot {
    void *ptr = nullptr;            // this device's address of `scratch`
    hipEvent_t done = nullptr;      // recorded after the last eager call
    hipStream_t last = nullptr;     // the stream of that call
    bool recorded = false;
};
StaticSlot g_static[kMaxDevices];
std::mutex g_static_mu;

}  // namespace
}  // namespace mi

static __device__ __align__(256) unsigned char scratch[mi::kStaticScratchBytes];

namespace mi {
namespace {

// The current device's slot, set up on its first call (the address of
// `scratch` and the event).  The caller holds g_static_mu.
mi_status static_slot(const char *fn, StaticSlot **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
    MI_REQUIRE(dev >= 0 && dev < kMaxDevices, MI_ERR_BAD_ARG, "%s: device %d beyond the %d this library tracks", fn,
               dev, kMaxDevices);
    StaticSlot &sl = g_static[dev];
    if (!sl.ptr) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MI_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d failed: %s", fn, dev,
                        hipGetErrorString(e));
        e = hipEventCreateWithFlags(&sl.done, hipEventDisableTiming);
        if (e != hipSuccess)
            return fail(MI_ERR_HIP, "%s: hipEventCreate on device %d failed: %s", fn, dev, hipGetErrorString(e));
        sl.ptr = ptr;
    }
    *out = &sl;
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status mi_decode_workspace_size(const mi_model_params *params, int m, size_t *bytes) {
    clear_error();
    mi_status st = check_model("mi_decode_workspace_size", params, m);
    if (st != MI_OK) return st;
    MI_REQUIRE(bytes, MI_ERR_NULL_POINTER, "mi_decode_workspace_size: bytes is NULL");
    *bytes = ws_layout(*params, m).total;
    return MI_OK;
}

extern "C" mi_status mi_decode_step(const mi_model_params *params, int m, const int64_t *ids, int64_t *next_ids,
                                    int32_t *logits, int ld_logits, int8_t *const *conv_state,
                                    int32_t *const *h_state, void *workspace, size_t workspace_bytes,
                                    void *stream) {
    clear_error();
    mi_status st = check_model("mi_decode_step", params, m);
    if (st != MI_OK) return st;
    const mi_model_params &p = *params;
    MI_REQUIRE(ids && next_ids && conv_state && h_state && workspace, MI_ERR_NULL_POINTER,
               "mi_decode_step: ids, next_ids, conv_state, h_state and workspace are required");
    MI_REQUIRE(aligned(workspace, kAlign), MI_ERR_BAD_ALIGNMENT, "mi_decode_step: workspace must be 256-byte aligned");
    const WsLayout w = ws_layout(p, m);
    MI_REQUIRE(workspace_bytes >= w.total, MI_ERR_BAD_ARG, "mi_decode_step: workspace of %zu bytes < %zu required",
               workspace_bytes, w.total);
    MI_REQUIRE(!logits || ld_logits >= p.vocab_size, MI_ERR_BAD_DIM, "mi_decode_step: ld_logits < vocab_size");
    for (int l = 0; l < p.n_layer; ++l)
        MI_REQUIRE(conv_state[l] && h_state[l], MI_ERR_NULL_POINTER, "mi_decode_step: state of layer %d is NULL", l);

    char *base = static_cast<char *>(workspace);
    int32_t *r = reinterpret_cast<int32_t *>(base + w.r);
    int64_t *stats = reinterpret_cast<int64_t *>(base + w.stats);
    int64_t *parts = reinterpret_cast<int64_t *>(base + w.parts);
    int8_t *xz = reinterpret_cast<int8_t *>(base + w.xz);
    int8_t *xs = reinterpret_cast<int8_t *>(base + w.xs);
    int8_t *yo = reinterpret_cast<int8_t *>(base + w.yo);
    int32_t *xpart = reinterpret_cast<int32_t *>(base + w.xpart);
    int64_t *keys = reinterpret_cast<int64_t *>(base + w.keys);
    const int d = p.d_model, D = (int)d_inner(p), N = p.d_state, R = p.dt_rank, nx = R + 2 * N;
    const int P = d / 16;  // row-statistics partials of the out_proj (one per 16 features)
    if (ssd(p))
        for (int l = 0; l < p.n_layer; ++l)
            MI_REQUIRE(p.layers[l].decay_tab, MI_ERR_NULL_POINTER, "mi_decode_step: decay_tab of layer %d is NULL", l);

    // every stage reports its own error; the first failure ends the step
#define MI_STEP(call)                    \
    do {                                 \
        const mi_status s_ = (call);     \
        if (s_ != MI_OK) return s_;      \
    } while (0)
    MI_STEP(mi_embed(ids, p.emb, r, m, d, p.vocab_size, stats, 1, stream));
    if (ssd(p)) {
        // MambaIntegerBlockV2 (spec section 7) in four kernels per layer: V2
        // norm + in_proj + conv step (row statistics as for the dyadic block),
        // x_proj, one block-scan step, out_proj with statistics partials
        int8_t *xp = reinterpret_cast<int8_t *>(base + w.xp);
        const int W = (int)ssd_xp_width(p);
        for (int l = 0; l < p.n_layer; ++l) {
            const mi_layer_params &ly = p.layers[l];
            MI_STEP(mi_norm_v2_in_proj_conv(r, l == 0 ? stats : parts, l == 0 ? 1 : P, ly.gamma, ly.w_in, ly.s_in,
                                            ly.conv_w, ly.conv_b, conv_state[l], xs, xz, m, d, D, stream));
            MI_STEP(mi_bitlinear_gemv(xs, D, ly.w_x, xp, W, MI_OUT_INT8, m, W, D, ly.s_x, 0, 0, 0, nullptr, 0.0f,
                                      nullptr, stream));
            MI_STEP(mi_ssd_block_scan(xs, xp, W, xz, 2 * D, D, ly.decay_tab, p.n_heads, ly.s_y, yo, h_state[l],
                                      h_state[l], m, 1, D, N, stream));
            MI_STEP(mi_bitlinear_residual_parts(yo, D, ly.w_out, r, d, m, d, D, ly.res_mult, ly.res_shift, ly.out_clamp, parts,
                                                stream));
        }
        MI_STEP(mi_norm_bitlinear_argmax(r, parts, P, p.gamma_f, p.w_head, logits, ld_logits, keys, m, p.vocab_size,
                                         d, stream));
        MI_STEP(mi_argmax_keys(keys, (p.vocab_size + 63) / 64, next_ids, m, stream));
        return MI_OK;
    }
    if (batched(p, m)) {
        int8_t *xp = reinterpret_cast<int8_t *>(base + w.xp);
        int8_t *a = reinterpret_cast<int8_t *>(base + w.a);
        int32_t *xq = quarters(p) ? reinterpret_cast<int32_t *>(base + w.xq) : nullptr;
        // logits rows at a 16-byte multiple stride in the workspace (the GEMV stores 16 bytes a lane)
        int32_t *lg = reinterpret_cast<int32_t *>(base + w.logits);
        const int ldl = (p.vocab_size + 3) / 4 * 4;
        const int W = (int)dyadic_xp_width(p);
        for (int l = 0; l < p.n_layer; ++l) {
            const mi_layer_params &ly = p.layers[l];
            if (l == 0) MI_STEP(mi_bitshift_norm(r, ly.gamma, a, m, d, stats, stream));
            else MI_STEP(mi_bitshift_norm_parts(r, ly.gamma, a, m, d, parts, P, 0, stream));
            MI_STEP(mi_bitlinear_gemv(a, d, ly.w_in, xz, 2 * D, MI_OUT_INT8, m, 2 * D, d, ly.s_in, 0, 0, 0, nullptr, 0.0f,
                                      nullptr, stream));
            if (quarters(p)) {
                MI_STEP(mi_conv_step_xpart(xz, 2 * D, ly.conv_w, ly.conv_b, conv_state[l], xs, ly.w_x, nx, xq, m, D,
                                           stream));
                MI_STEP(mi_xpart_dt_scan_step(xq, 4, ly.s_x, R, ly.w_dt, ly.s_dt, xs, xz, 2 * D, D, ly.base,
                                              ly.decay_shift, ly.s_y, h_state[l], yo, m, D, N, stream));
            } else {
                MI_STEP(mi_conv_step_xproj(xz, 2 * D, ly.conv_w, ly.conv_b, conv_state[l], xs, ly.w_x, ly.s_x, nx, xp,
                                           W, m, D, stream));
                MI_STEP(mi_dt_scan_step(xp, W, R, ly.w_dt, ly.s_dt, xs, xz, 2 * D, D, ly.base, ly.decay_shift, ly.s_y,
                                        h_state[l], yo, m, D, N, stream));
            }
            MI_STEP(mi_bitlinear_residual_parts(yo, D, ly.w_out, r, d, m, d, D, ly.res_mult, ly.res_shift, ly.out_clamp, parts,
                                                stream));
        }
        MI_STEP(mi_bitshift_norm_parts(r, p.gamma_f, a, m, d, parts, P, 0, stream));
        MI_STEP(mi_bitlinear_gemv(a, d, p.w_head, lg, ldl, MI_OUT_INT32, m, p.vocab_size, d, 0, 0, 0, 0, nullptr, 0.0f,
                                  nullptr, stream));
        MI_STEP(mi_argmax_i32(lg, ldl, next_ids, m, p.vocab_size, stream));
        if (logits) {
            const hipError_t e = hipMemcpy2DAsync(logits, (size_t)ld_logits * 4, lg, (size_t)ldl * 4,
                                                  (size_t)p.vocab_size * 4, (size_t)m, hipMemcpyDeviceToDevice,
                                                  as_stream(stream));
            if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_decode_step: logits copy failed: %s", hipGetErrorString(e));
        }
        return MI_OK;
    }
    for (int l = 0; l < p.n_layer; ++l) {
        const mi_layer_params &ly = p.layers[l];
        // layer 0 reads the embedding's full sums, later layers the partials
        // of the previous out_proj (one buffer: each norm reads it before its
        // layer's out_proj rewrites it, in stream order)
        MI_STEP(mi_norm_in_proj_conv_xpart(r, l == 0 ? stats : parts, l == 0 ? 1 : P, ly.gamma, ly.w_in, ly.s_in,
                                           ly.conv_w, ly.conv_b, conv_state[l], xs, xz, ly.w_x, nx, xpart, m, d, D,
                                           stream));
        MI_STEP(mi_xpart_dt_scan_step(xpart, D / 16, ly.s_x, R, ly.w_dt, ly.s_dt, xs, xz, 2 * D, D, ly.base,
                                      ly.decay_shift, ly.s_y, h_state[l], yo, m, D, N, stream));
        MI_STEP(mi_bitlinear_residual_parts(yo, D, ly.w_out, r, d, m, d, D, ly.res_mult, ly.res_shift, ly.out_clamp, parts,
                                            stream));
    }
    MI_STEP(mi_norm_bitlinear_argmax(r, parts, P, p.gamma_f, p.w_head, logits, ld_logits, keys, m, p.vocab_size, d,
                                     stream));
    MI_STEP(mi_argmax_keys(keys, (p.vocab_size + 63) / 64, next_ids, m, stream));
#undef MI_STEP
    return MI_OK;
}


extern "C" mi_status mi_decode_step_static(const mi_model_params *params, int m, const int64_t *ids,
                                           int64_t *next_ids, int32_t *logits, int ld_logits,
                                           int8_t *const *conv_state, int32_t *const *h_state, void *stream) {
    clear_error();
    mi_status st = check_model("mi_decode_step_static", params, m);
    if (st != MI_OK) return st;
    const size_t need = ws_layout(*params, m).total;
    MI_REQUIRE(need <= kStaticScratchBytes, MI_ERR_BAD_DIM,
               "mi_decode_step_static: this model at m=%d needs %zu bytes of workspace; the static scratch holds %zu "
               "(call mi_decode_step with a workspace of your own)", m, need, kStaticScratchBytes);
    MI_REQUIRE(ids && next_ids && conv_state && h_state, MI_ERR_NULL_POINTER,
               "mi_decode_step_static: ids, next_ids, conv_state and h_state are required");
    std::lock_guard<std::mutex> lock(g_static_mu);
    StaticSlot *sl = nullptr;
    st = static_slot("mi_decode_step_static", &sl);
    if (st != MI_OK) return st;
    const hipStream_t s = as_stream(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess)
        return fail(MI_ERR_HIP, "mi_decode_step_static: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    const bool capturing = cap != hipStreamCaptureStatusNone;
    if (!capturing && sl->recorded && sl->last != s) {
        e = hipEventQuery(sl->done);
        MI_REQUIRE(e != hipErrorNotReady, MI_ERR_BAD_ARG,
                   "mi_decode_step_static: the previous call, on another stream, is still running and holds the "
                   "static workspace (order the calls: one stream, or wait for the other)");
        if (e != hipSuccess)
            return fail(MI_ERR_HIP, "mi_decode_step_static: hipEventQuery failed: %s", hipGetErrorString(e));
    }
    st = mi_decode_step(params, m, ids, next_ids, logits, ld_logits, conv_state, h_state, sl->ptr, kStaticScratchBytes,
                        stream);
    if (st == MI_OK && !capturing) {
        e = hipEventRecord(sl->done, s);
        if (e != hipSuccess)
            return fail(MI_ERR_HIP, "mi_decode_step_static: hipEventRecord failed: %s", hipGetErrorString(e));
        sl->last = s;
        sl->recorded = true;
    }
    return st;
}
