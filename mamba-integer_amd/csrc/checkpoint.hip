// Integer checkpoint, formats 1 (spec mi-spec-1) and 2 (spec mi-spec-2):
// reader, validation and upload into one caller-owned device buffer.  The
// two formats share one layout; format 2 gives the last per-layer scalar a
// meaning (the SSD block's out_proj accumulator bound, spec rule 7.9), which
// format 1 holds as zero (no bound, as mi-spec-1 computes).
//
// The reference's inference export (scripts/export_int8.py:50-135) writes a
// bare 0xDAD1C stream (float embedding, conv and gains, one int8 byte per
// ternary weight, float scales) that only the exact same loop can read back,
// and its loader (src/cpp_engine/mamba_infer.cpp:46-118) exit()s on any
// error and cudaMallocs every tensor.  Here the file is a table of named,
// typed, shaped tensors, each at a 256-byte aligned offset with its CRC-32,
// holding the integer parameters themselves (2-bit packed ternary matrices,
// int8 embedding and taps, int32 decays, the per-layer shifts); every check
// reports an mi_status, and the upload fills a buffer the caller allocated.
//
// File layout (little-endian):
//   header, 128 bytes: magic "MIQCKPT\0", u32 format (1 or 2), u32 header
//     bytes (128), char spec[16] ("mi-spec-1" / "mi-spec-2"), u32 d_model, n_layer, vocab_size,
//     d_state, dt_rank, u32 tensor count, u64 table offset, u64 file bytes,
//     f32 logit_scale, u32 CRC-32 of the table, u32 block (0 dyadic scan,
//     1 multi-head SSD), u32 n_heads, u32 d_head, zeros;
//   table: one 96-byte entry per tensor: char name[48] (NUL-padded), u32
//     dtype (1 i8, 2 u8, 3 i16, 4 i32, 5 f32), u32 ndim, u32 shape[4], u64
//     offset, u64 bytes, u32 CRC-32 of the bytes, u32 zero;
//   data: each tensor at its offset (a multiple of 256), zero padding between.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "mi_common.hpp"

struct mi_checkpoint {
    mi_checkpoint_info info;
    std::vector<uint8_t> bytes;  // the whole file, validated
    struct Tensor {
        uint32_t dtype, ndim;
        uint64_t shape[4];
        uint64_t offset, nbytes;
    };
    std::map<std::string, Tensor> tensors;
    std::vector<int32_t> scalars;  // [n_layer][8]
};

namespace mi {
namespace {

constexpr char kMagic[8] = {'M', 'I', 'Q', 'C', 'K', 'P', 'T', '\0'};
constexpr uint32_t kFormatMin = 1, kFormatMax = 2;
constexpr size_t kHeaderBytes = 128, kEntryBytes = 96, kDataAlign = 256;
constexpr int kScalars = 8;  // s_in, s_x, s_dt, decay_shift, s_y, res_mult, res_shift, out_clamp
enum { kI8 = 1, kU8 = 2, kI16 = 3, kI32 = 4, kF32 = 5 };

uint32_t crc32_ieee(const uint8_t *p, size_t n) {
    static uint32_t table[256];
    static bool ready = false;
    if (!ready) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
        ready = true;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; ++i) c = table[(c ^ p[i]) & 0xFF] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

template <typename T>
T rd(const uint8_t *p) {
    T v;
    memcpy(&v, p, sizeof(T));
    return v;
}

size_t elem_bytes(uint32_t dtype) {
    switch (dtype) {
        case kI8: case kU8: return 1;
        case kI16: return 2;
        case kI32: case kF32: return 4;
        default: return 0;
    }
}

struct Want {
    std::string name;
    uint32_t dtype;
    std::vector<uint64_t> shape;
};

uint64_t ssd_xp_width(const mi_checkpoint_info &in) {
    return ((uint64_t)2 * in.n_heads * in.d_state + in.n_heads + 15) / 16 * 16;
}

// The tensors a format-1 file holds for the given dims, in canonical order
// (the device layout of mi_checkpoint_upload follows this order).
std::vector<Want> expected(const mi_checkpoint_info &in) {
    const bool ssd = in.block == MI_BLOCK_SSD;
    const uint64_t d = in.d_model, D = ssd ? (uint64_t)in.n_heads * in.d_head : 2 * d, N = in.d_state,
                   R = in.dt_rank, V = in.vocab_size;
    std::vector<Want> w;
    w.push_back({"emb", kI8, {V, d}});
    w.push_back({"gamma_f", kI16, {d}});
    w.push_back({"w_head", kU8, {V, d / 4}});
    w.push_back({"layer_scalars", kI32, {(uint64_t)in.n_layer, kScalars}});
    for (int l = 0; l < in.n_layer; ++l) {
        const std::string p = "layers." + std::to_string(l) + ".";
        w.push_back({p + "gamma", kI16, {d}});
        w.push_back({p + "w_in", kU8, {2 * D, d / 4}});
        w.push_back({p + "conv_w", kI8, {D, 4}});
        w.push_back({p + "conv_b", kI32, {D}});
        if (ssd) {
            w.push_back({p + "w_x", kU8, {ssd_xp_width(in), D / 4}});
            w.push_back({p + "decay_tab", kI32, {(uint64_t)in.n_heads, 255}});
        } else {
            w.push_back({p + "w_x", kU8, {R + 2 * N, D / 4}});
            w.push_back({p + "w_dt", kU8, {D, R / 4}});
            w.push_back({p + "base", kI32, {D, N}});
        }
        w.push_back({p + "w_out", kU8, {d, D / 4}});
    }
    return w;
}

size_t up256(size_t v) { return (v + kDataAlign - 1) / kDataAlign * kDataAlign; }

// A packed ternary byte holds four 2-bit codes; code 0b10 is never written.
bool packed_ok(const uint8_t *p, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        if (((p[i] >> 1) & ~p[i] & 0x55) != 0) return false;
    return true;
}

mi_status parse(mi_checkpoint &ck, const char *path) {
    const std::vector<uint8_t> &b = ck.bytes;
    MI_REQUIRE(b.size() >= kHeaderBytes, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: %zu bytes, shorter than the header",
               path, b.size());
    MI_REQUIRE(memcmp(b.data(), kMagic, 8) == 0, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: not an integer checkpoint "
               "(bad magic)", path);
    const uint32_t format = rd<uint32_t>(&b[8]), hbytes = rd<uint32_t>(&b[12]);
    MI_REQUIRE(format >= kFormatMin && format <= kFormatMax, MI_ERR_BAD_ARG,
               "mi_checkpoint_open: %s: format %u (this library reads %u to %u)", path, format, kFormatMin, kFormatMax);
    MI_REQUIRE(hbytes == kHeaderBytes, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: header of %u bytes", path, hbytes);
    mi_checkpoint_info &in = ck.info;
    memset(&in, 0, sizeof(in));
    in.format_version = (int)format;
    memcpy(in.spec, &b[16], 16);
    in.spec[15] = '\0';
    const char *want_spec = format == 1 ? "mi-spec-1" : "mi-spec-2";
    MI_REQUIRE(strcmp(in.spec, want_spec) == 0, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: spec '%s' in a format-%u "
               "file (expected %s)", path, in.spec, format, want_spec);
    const uint32_t dm = rd<uint32_t>(&b[32]), nl = rd<uint32_t>(&b[36]), vs = rd<uint32_t>(&b[40]),
                   ds = rd<uint32_t>(&b[44]), dr = rd<uint32_t>(&b[48]), nt = rd<uint32_t>(&b[52]);
    const uint64_t toff = rd<uint64_t>(&b[56]), fbytes = rd<uint64_t>(&b[64]);
    in.logit_scale = rd<float>(&b[72]);
    const uint32_t tcrc = rd<uint32_t>(&b[76]);
    const uint32_t blk = rd<uint32_t>(&b[80]), nh = rd<uint32_t>(&b[84]), dh = rd<uint32_t>(&b[88]);
    MI_REQUIRE(fbytes == b.size(), MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: header says %llu bytes, file has %zu",
               path, (unsigned long long)fbytes, b.size());
    MI_REQUIRE(blk == MI_BLOCK_DYADIC || blk == MI_BLOCK_SSD, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: block %u "
               "unknown", path, blk);
    const bool ssd = blk == MI_BLOCK_SSD;
    MI_REQUIRE(dm >= 16 && dm % 16 == 0 && dm <= 65536 && nl >= 1 && nl <= 4096 && vs >= 1 && vs <= (1u << 24) &&
                   ds >= 1 && ds <= 64 &&
                   (ssd ? (nh >= 1 && nh <= 1024 && dh >= 16 && dh % 16 == 0 && dh <= 4096 &&
                           (ds == 16 || ds == 32 || ds == 64))
                        : (dr >= 16 && dr % 16 == 0 && dr <= 4096)),
               MI_ERR_BAD_DIM, "mi_checkpoint_open: %s: dims d_model=%u n_layer=%u vocab=%u d_state=%u dt_rank=%u "
               "n_heads=%u d_head=%u outside the format's limits", path, dm, nl, vs, ds, dr, nh, dh);
    in.d_model = (int)dm; in.n_layer = (int)nl; in.vocab_size = (int)vs; in.d_state = (int)ds; in.dt_rank = (int)dr;
    in.block = (int)blk; in.n_heads = ssd ? (int)nh : 0; in.d_head = ssd ? (int)dh : 0;
    MI_REQUIRE(in.logit_scale > 0.0f, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: logit_scale must be positive", path);
    // range checks are written as subtractions so that no sum of header fields can wrap
    const uint64_t size = b.size();
    MI_REQUIRE(toff >= kHeaderBytes && toff <= size && (uint64_t)nt <= (size - toff) / kEntryBytes, MI_ERR_BAD_ARG,
               "mi_checkpoint_open: %s: tensor table outside the file", path);
    const uint64_t table_end = toff + (uint64_t)nt * kEntryBytes;
    MI_REQUIRE(crc32_ieee(&b[toff], (size_t)nt * kEntryBytes) == tcrc, MI_ERR_BAD_ARG,
               "mi_checkpoint_open: %s: tensor table CRC mismatch", path);

    for (uint32_t i = 0; i < nt; ++i) {
        const uint8_t *e = &b[toff + (size_t)i * kEntryBytes];
        char name[49];
        memcpy(name, e, 48);
        name[48] = '\0';
        mi_checkpoint::Tensor t{};
        t.dtype = rd<uint32_t>(e + 48);
        t.ndim = rd<uint32_t>(e + 52);
        for (int j = 0; j < 4; ++j) t.shape[j] = rd<uint32_t>(e + 56 + 4 * j);
        t.offset = rd<uint64_t>(e + 72);
        t.nbytes = rd<uint64_t>(e + 80);
        const uint32_t crc = rd<uint32_t>(e + 88);
        MI_REQUIRE(strnlen(name, 48) < 48, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: tensor %u name not terminated",
                   path, i);
        MI_REQUIRE(t.ndim >= 1 && t.ndim <= 4 && elem_bytes(t.dtype) != 0, MI_ERR_BAD_ARG,
                   "mi_checkpoint_open: %s: tensor '%s': dtype %u / ndim %u invalid", path, name, t.dtype, t.ndim);
        uint64_t count = 1;
        bool fits = true;
        for (uint32_t j = 0; j < t.ndim; ++j) {
            fits = fits && (t.shape[j] == 0 || count <= UINT64_MAX / 8 / t.shape[j]);
            count *= t.shape[j];
        }
        MI_REQUIRE(fits && t.nbytes == count * elem_bytes(t.dtype), MI_ERR_BAD_ARG,
                   "mi_checkpoint_open: %s: tensor '%s': %llu bytes for its shape", path, name,
                   (unsigned long long)t.nbytes);
        MI_REQUIRE(t.offset % kDataAlign == 0 && t.offset >= table_end && t.offset <= size &&
                       t.nbytes <= size - t.offset,
                   MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: tensor '%s' at offset %llu: misaligned or outside the "
                   "file", path, name, (unsigned long long)t.offset);
        MI_REQUIRE(crc32_ieee(&b[t.offset], (size_t)t.nbytes) == crc, MI_ERR_BAD_ARG,
                   "mi_checkpoint_open: %s: tensor '%s': CRC mismatch (corrupted data)", path, name);
        MI_REQUIRE(ck.tensors.emplace(name, t).second, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: tensor '%s' twice",
                   path, name);
    }
    size_t dev = 0;
    for (const Want &w : expected(in)) {
        auto it = ck.tensors.find(w.name);
        MI_REQUIRE(it != ck.tensors.end(), MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: tensor '%s' missing", path,
                   w.name.c_str());
        const mi_checkpoint::Tensor &t = it->second;
        bool same = t.dtype == w.dtype && t.ndim == w.shape.size();
        for (size_t j = 0; same && j < w.shape.size(); ++j) same = t.shape[j] == w.shape[j];
        MI_REQUIRE(same, MI_ERR_BAD_DIM, "mi_checkpoint_open: %s: tensor '%s': dtype or shape does not match the "
                   "dims", path, w.name.c_str());
        if (t.dtype == kU8)
            MI_REQUIRE(packed_ok(&b[t.offset], t.nbytes), MI_ERR_BAD_ARG,
                       "mi_checkpoint_open: %s: tensor '%s' holds the invalid ternary code 0b10", path,
                       w.name.c_str());
        dev += up256((size_t)t.nbytes);
    }
    MI_REQUIRE(ck.tensors.size() == expected(in).size(), MI_ERR_BAD_ARG,
               "mi_checkpoint_open: %s: %zu tensors, the format holds %zu", path, ck.tensors.size(),
               expected(in).size());
    in.device_bytes = dev;

    const mi_checkpoint::Tensor &sc = ck.tensors["layer_scalars"];
    ck.scalars.resize((size_t)nl * kScalars);
    memcpy(ck.scalars.data(), &b[sc.offset], sc.nbytes);
    for (uint32_t l = 0; l < nl; ++l) {
        const int32_t *s = &ck.scalars[(size_t)l * kScalars];
        MI_REQUIRE(s[0] >= 0 && s[0] <= 30 && s[1] >= 0 && s[1] <= 30 && s[2] >= 0 && s[2] <= 30 && s[4] >= 0 &&
                       s[4] <= 30 && s[6] >= 0 && s[6] <= 62,
                   MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: layer %u: a requant shift is outside its range", path, l);
        MI_REQUIRE(s[3] == 15, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: layer %u: decay shift %d (the scan kernels "
                   "take 15)", path, l, s[3]);
        // out_clamp: zero in format 1 and in dyadic-block layers (no bound);
        // a format-2 SSD layer carries its bound, >= 1
        if (format == 1 || !ssd)
            MI_REQUIRE(s[7] == 0, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: layer %u: out_clamp %d where the format "
                       "or block has none", path, l, s[7]);
        else
            MI_REQUIRE(s[7] >= 1, MI_ERR_BAD_ARG, "mi_checkpoint_open: %s: layer %u: out_clamp %d must be >= 1",
                       path, l, s[7]);
        // decay numerators: clamp(base + dm) of the dyadic block needs base in
        // [0, 32000]; the SSD block's table entries are used as they are
        const int32_t hi = ssd ? 32768 : 32000;
        const mi_checkpoint::Tensor &bt = ck.tensors["layers." + std::to_string(l) + (ssd ? ".decay_tab" : ".base")];
        const int32_t *base = reinterpret_cast<const int32_t *>(&b[bt.offset]);
        for (uint64_t i = 0; i < bt.nbytes / 4; ++i)
            MI_REQUIRE(base[i] >= 0 && base[i] <= hi, MI_ERR_BAD_ARG,
                       "mi_checkpoint_open: %s: layer %u: decay numerator %d outside [0,%d]", path, l, base[i], hi);
    }
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status mi_checkpoint_open(const char *path, mi_checkpoint **out) {
    clear_error();
    MI_REQUIRE(path && out, MI_ERR_NULL_POINTER, "mi_checkpoint_open: path and out are required");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    MI_REQUIRE(f, MI_ERR_BAD_ARG, "mi_checkpoint_open: cannot open %s", path);
    mi_checkpoint *ck = new mi_checkpoint();
    fseek(f, 0, SEEK_END);
    const long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    bool ok = size >= 0;
    if (ok) {
        ck->bytes.resize((size_t)size);
        ok = size == 0 || fread(ck->bytes.data(), 1, (size_t)size, f) == (size_t)size;
    }
    fclose(f);
    if (!ok) {
        delete ck;
        return fail(MI_ERR_BAD_ARG, "mi_checkpoint_open: cannot read %s", path);
    }
    const mi_status st = parse(*ck, path);
    if (st != MI_OK) {
        delete ck;
        return st;
    }
    *out = ck;
    return MI_OK;
}

extern "C" mi_status mi_checkpoint_get_info(const mi_checkpoint *ck, mi_checkpoint_info *info) {
    clear_error();
    MI_REQUIRE(ck && info, MI_ERR_NULL_POINTER, "mi_checkpoint_get_info: checkpoint and info are required");
    *info = ck->info;
    return MI_OK;
}

extern "C" mi_status mi_checkpoint_upload(const mi_checkpoint *ck, void *device, size_t device_bytes,
                                          mi_model_params *params, mi_layer_params *layers, int n_layers,
                                          void *stream) {
    clear_error();
    MI_REQUIRE(ck && device && params && layers, MI_ERR_NULL_POINTER,
               "mi_checkpoint_upload: checkpoint, device, params and layers are required");
    const mi_checkpoint_info &in = ck->info;
    MI_REQUIRE(n_layers == in.n_layer, MI_ERR_BAD_DIM, "mi_checkpoint_upload: layers holds %d entries, the model %d",
               n_layers, in.n_layer);
    MI_REQUIRE(aligned(device, kDataAlign), MI_ERR_BAD_ALIGNMENT, "mi_checkpoint_upload: device must be 256-byte "
               "aligned");
    MI_REQUIRE(device_bytes >= in.device_bytes, MI_ERR_BAD_ARG, "mi_checkpoint_upload: %zu device bytes < %zu "
               "required", device_bytes, in.device_bytes);
    hipStream_t hs = as_stream(stream);
    char *dev = static_cast<char *>(device);
    std::map<std::string, const void *> where;
    size_t off = 0;
    for (const Want &w : expected(in)) {
        const mi_checkpoint::Tensor &t = ck->tensors.at(w.name);
        const hipError_t e = hipMemcpyAsync(dev + off, &ck->bytes[t.offset], (size_t)t.nbytes,
                                            hipMemcpyHostToDevice, hs);
        if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_checkpoint_upload: copy of '%s': %s", w.name.c_str(),
                                         hipGetErrorString(e));
        where[w.name] = dev + off;
        off += up256((size_t)t.nbytes);
    }
    const hipError_t e = hipStreamSynchronize(hs);
    if (e != hipSuccess) return fail(MI_ERR_HIP, "mi_checkpoint_upload: %s", hipGetErrorString(e));

    params->d_model = in.d_model;
    params->n_layer = in.n_layer;
    params->vocab_size = in.vocab_size;
    params->d_state = in.d_state;
    params->dt_rank = in.dt_rank;
    params->emb = static_cast<const int8_t *>(where["emb"]);
    params->gamma_f = static_cast<const int16_t *>(where["gamma_f"]);
    params->w_head = static_cast<const uint8_t *>(where["w_head"]);
    params->layers = layers;
    params->block = in.block;
    params->n_heads = in.n_heads;
    params->d_head = in.d_head;
    const bool ssd = in.block == MI_BLOCK_SSD;
    for (int l = 0; l < in.n_layer; ++l) {
        const std::string p = "layers." + std::to_string(l) + ".";
        const int32_t *s = &ck->scalars[(size_t)l * kScalars];
        mi_layer_params &ly = layers[l];
        ly.gamma = static_cast<const int16_t *>(where[p + "gamma"]);
        ly.w_in = static_cast<const uint8_t *>(where[p + "w_in"]);
        ly.s_in = s[0];
        ly.conv_w = static_cast<const int8_t *>(where[p + "conv_w"]);
        ly.conv_b = static_cast<const int32_t *>(where[p + "conv_b"]);
        ly.w_x = static_cast<const uint8_t *>(where[p + "w_x"]);
        ly.s_x = s[1];
        ly.w_dt = ssd ? nullptr : static_cast<const uint8_t *>(where[p + "w_dt"]);
        ly.s_dt = s[2];
        ly.base = ssd ? nullptr : static_cast<const int32_t *>(where[p + "base"]);
        ly.decay_tab = ssd ? static_cast<const int32_t *>(where[p + "decay_tab"]) : nullptr;
        ly.decay_shift = s[3];
        ly.s_y = s[4];
        ly.w_out = static_cast<const uint8_t *>(where[p + "w_out"]);
        ly.res_mult = s[5];
        ly.res_shift = s[6];
        ly.out_clamp = s[7];
    }
    return MI_OK;
}

extern "C" void mi_checkpoint_close(mi_checkpoint *ck) { delete ck; }
