"""Integer checkpoints (format 2, and format-1 files) and the float state-dict converter, on the
CPU: the Python writer/reader, the native reader (mi_checkpoint_open, no
device calls), and the conversion rules pinned by closed forms and hand-made
rounding ties (the reference's float model is not run here)."""
import ctypes
import math
import struct
import zlib

import numpy as np
import pytest

from mamba_int import ModelDims, checkpoint as ckpt, init_random_params, pack_ternary, unpack_ternary

DIMS = ModelDims(d_model=64, n_layer=2, vocab_size=100, d_state=16, dt_rank=16)


def _params():
    return init_random_params(ModelDims(**DIMS.__dict__), 4)


def _equal(p, q):
    assert p.dims == q.dims
    for k in ("emb", "gamma_f", "w_head"):
        assert np.array_equal(getattr(p, k), getattr(q, k)), k
    for a, b in zip(p.layers, q.layers):
        for k in a.__dataclass_fields__:
            assert np.array_equal(getattr(a, k), getattr(b, k)), k


def _native_open(path):
    from mamba_int import _lib
    h = ctypes.c_void_p()
    st = _lib.raw("mi_checkpoint_open", str(path).encode(), ctypes.byref(h))
    if st == 0:
        _lib.load().mi_checkpoint_close(h)
    return st, _lib.last_error()


def test_round_trip_and_layout(tmp_path):
    from mamba_int.native import NativeCheckpoint
    p = _params()
    path = tmp_path / "m.miq"
    ckpt.save(p, str(path), 0.0125)
    q, scale = ckpt.load(str(path))
    _equal(p, q)
    assert scale == np.float32(0.0125)
    b = path.read_bytes()
    magic, fmt, hb, spec, d, nl, v, ns, dr, nt, toff, fb, ls, tcrc, blk, nh, dh = ckpt._HEADER.unpack_from(b, 0)
    assert (blk, nh, dh) == (0, 0, 0)
    assert (magic, fmt, hb, spec.rstrip(b"\0"), fb) == (b"MIQCKPT\0", 2, 128, b"mi-spec-2", len(b))
    assert (d, nl, v, ns, dr) == (64, 2, 100, 16, 16) and nt == 4 + 8 * 2
    assert zlib.crc32(b[toff:toff + 96 * nt]) == tcrc
    for i in range(nt):
        e = ckpt._ENTRY.unpack_from(b, toff + 96 * i)
        off, nbytes, crc = e[7], e[8], e[9]
        assert off % 256 == 0 and zlib.crc32(b[off:off + nbytes]) == crc
    # the native reader agrees on the header and on the device layout size
    ck = NativeCheckpoint(str(path))
    i = ck.info
    assert (i.format_version, i.spec, i.d_model, i.n_layer, i.vocab_size, i.d_state, i.dt_rank) == \
        (2, b"mi-spec-2", 64, 2, 100, 16, 16)
    assert i.logit_scale == np.float32(0.0125)
    assert i.device_bytes == sum(-(-a.nbytes // 256) * 256 for a in ckpt._tensors(p).values())


def _rewrite(path, name, fn):
    """Applies fn to tensor `name`'s bytes and rewrites its CRC (and the table's)."""
    b = bytearray(path.read_bytes())
    toff, nt = struct.unpack_from("<Q", b, 56)[0], struct.unpack_from("<I", b, 52)[0]
    for i in range(nt):
        at = toff + 96 * i
        e = list(ckpt._ENTRY.unpack_from(b, at))
        if e[0].rstrip(b"\0").decode() == name:
            off, n = e[7], e[8]
            b[off:off + n] = fn(bytes(b[off:off + n]))
            e[9] = zlib.crc32(bytes(b[off:off + n]))
            ckpt._ENTRY.pack_into(b, at, *e)
    struct.pack_into("<I", b, 76, zlib.crc32(bytes(b[toff:toff + 96 * nt])))
    path.write_bytes(bytes(b))


def _flip(b):
    return b[:3] + bytes([b[3] ^ 1]) + b[4:]


@pytest.mark.parametrize("case,needle", [
    ("magic", "magic"), ("truncated", "bytes"), ("data", "CRC mismatch"), ("table", "table CRC"),
    ("spec", "spec"), ("code", "0b10"), ("shift", "decay shift"), ("base", "decay numerator"),
    ("shape", "does not match"),
])
def test_corrupt_files_are_rejected(tmp_path, case, needle):
    """Both readers refuse each kind of damage with a message naming it."""
    p = _params()
    path = tmp_path / "m.miq"
    if case == "code":
        p.layers[1].w_in[3, 2] = 0x02          # 2-bit code 0b10 in a packed byte
    if case == "shift":
        p.layers[0].k = 14
    if case == "base":
        p.layers[1].base[0, 0] = 32001
    ckpt.save(p, str(path), 1.0)
    b = bytearray(path.read_bytes())
    if case == "magic":
        b[0] = ord("X")
    elif case == "truncated":
        b = b[:-100]
    elif case == "data":
        b[-5] ^= 0x40
    elif case == "table":
        b[128 + 3] ^= 1
    elif case == "spec":
        b[16 + 8] = ord("9")
    if case in ("magic", "truncated", "data", "table", "spec"):
        path.write_bytes(bytes(b))
    if case == "shape":                         # a tensor whose shape disagrees with the dims
        bb = bytearray(path.read_bytes())
        toff = struct.unpack_from("<Q", bb, 56)[0]
        struct.pack_into("<II", bb, toff + 56, 50, 128)      # emb [100, 64] -> [50, 128]: same bytes
        struct.pack_into("<I", bb, 76, zlib.crc32(bytes(bb[toff:toff + 96 * 20])))
        path.write_bytes(bytes(bb))
    with pytest.raises(ckpt.CheckpointError, match=needle):
        ckpt.load(str(path))
    st, msg = _native_open(path)
    assert st != 0 and needle in msg, msg


@pytest.mark.parametrize("nt", [200_000, 40_000_000])
def test_wrapping_table_offset_is_rejected(tmp_path, nt):
    """A table offset chosen so that offset + count * 96 wraps past 2^64 to a
    small number is refused as outside the file, before any byte of the table
    is read (the CRC pass would otherwise read far outside the buffer)."""
    p = _params()
    path = tmp_path / "m.miq"
    ckpt.save(p, str(path), 1.0)
    b = bytearray(path.read_bytes())
    struct.pack_into("<I", b, 52, nt)
    struct.pack_into("<Q", b, 56, (1 << 64) - nt * 96 + 128)
    path.write_bytes(bytes(b))
    with pytest.raises(ckpt.CheckpointError, match="outside the file"):
        ckpt.load(str(path))
    st, msg = _native_open(path)
    assert st != 0 and "outside the file" in msg, msg


@pytest.mark.parametrize("what", ["offset", "shape"])
def test_wrapping_tensor_entry_is_rejected(tmp_path, what):
    """A table entry whose offset + bytes, or whose shape product, wraps past
    2^64 is refused (the table CRC is rewritten, so only the range checks stand
    in the way)."""
    p = _params()
    path = tmp_path / "m.miq"
    ckpt.save(p, str(path), 1.0)
    b = bytearray(path.read_bytes())
    toff, nt = struct.unpack_from("<Q", b, 56)[0], struct.unpack_from("<I", b, 52)[0]
    e = list(ckpt._ENTRY.unpack_from(b, toff))
    if what == "offset":
        e[7] = (1 << 64) - 256                   # offset + bytes wraps to bytes - 256
        needle = "outside the file"
    else:
        e[2], e[3:7] = 4, [1 << 31, 1 << 31, 1 << 31, 1 << 3]   # product 2^96 wraps to 0
        e[8] = 0
        needle = "bytes for its shape"
    ckpt._ENTRY.pack_into(b, toff, *e)
    struct.pack_into("<I", b, 76, zlib.crc32(bytes(b[toff:toff + 96 * nt])))
    path.write_bytes(bytes(b))
    with pytest.raises(ckpt.CheckpointError, match=needle):
        ckpt.load(str(path))
    st, msg = _native_open(path)
    assert st != 0 and needle in msg, msg


def test_rewritten_tensor_with_valid_crc_loads(tmp_path):
    """_rewrite (used to plant damage behind valid CRCs) keeps a file valid when
    it changes nothing, and the readers see a changed but valid byte."""
    p = _params()
    path = tmp_path / "m.miq"
    ckpt.save(p, str(path), 1.0)
    _rewrite(path, "layers.0.conv_b", _flip)
    q, _ = ckpt.load(str(path))
    assert q.layers[0].conv_b[0] == p.layers[0].conv_b[0] ^ (1 << 24)
    assert _native_open(path)[0] == 0


# ------------------------------------------------------------------ converter
def test_ternary_rounds_half_to_even():
    """weight_quant_ternary (rational_bitnet.py:63-85): mean|W| = 1 exactly, so
    W / s = W; ties 0.5 -> 0, 1.5 -> 2 -> 1, 2.5 -> 2 -> 1 (half to even)."""
    w = np.array([[0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.0, 1.0, 0.0, 0.0]], np.float32)
    q, s = ckpt.ternary(w)
    assert s == 1.0
    assert q.tolist() == [[0, 0, 1, -1, 1, -1, 0, 1, 0, 0]]
    q, s = ckpt.ternary(np.zeros((2, 16), np.float32))      # the 1e-6 floor of the scale
    assert s == np.float32(1e-6) and not q.any()


def test_shift_rules_closed_forms():
    assert ckpt.requant_shift_for(2.0 ** -5, 4, 4) == 5
    assert ckpt.requant_shift_for(2.0 ** -5 * 1.40, 4, 4) == 5       # log2 = -4.51 -> 5
    assert ckpt.requant_shift_for(2.0 ** -5 * 1.42, 4, 4) == 4       # -4.49 -> 4
    assert ckpt.requant_shift_for(2.0 ** -5, 4, 0) == 9              # Q4 -> Q0: 4 more
    assert ckpt.requant_shift_for(8.0, 4, 4) == 0                    # clamped at 0
    for s, g in ((0.03, 0.144), (0.011, -0.2), (2.0 ** -7, 1.0)):
        mult, shift = ckpt.residual_factor(s, g)
        f = 16 * s * g
        assert 2 ** 14 <= abs(mult) <= 2 ** 15
        assert abs(mult / 2.0 ** shift - f) <= 2.0 ** -(shift + 1) + 1e-18
    assert ckpt.residual_factor(0.03, 0.0) == (0, 0)


def _state_dict(rng, dims=DIMS, **over):
    import torch
    d, D, N, R, V = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank, dims.vocab_size
    f = lambda *s, sc=1.0: torch.from_numpy((rng.standard_normal(s) * sc).astype(np.float32))  # noqa: E731
    sd = {"embedding.weight": f(V, d), "norm_f.gamma": 1 + f(d, sc=0.1), "norm_f.step_size": torch.ones(1),
          "lm_head.weight": f(V, d, sc=d ** -1)}
    for i in range(dims.n_layer):
        p = f"layers.{i}."
        sd.update({p + "norm.gamma": 1 + f(d, sc=0.1), p + "norm.step_size": torch.tensor([0.75]),
                   p + "in_proj.weight": f(2 * D, d, sc=d ** -0.5), p + "conv1d.weight": f(D, 1, 4, sc=0.5),
                   p + "conv1d.bias": f(D, sc=0.1), p + "x_proj.weight": f(R + 2 * N, D, sc=D ** -0.5),
                   p + "dt_proj.weight": f(D, R, sc=R ** -0.5), p + "out_proj.weight": f(d, D, sc=D ** -0.5),
                   p + "base_decay_nums": torch.from_numpy(rng.uniform(-50, 33000, (D, N)).astype(np.float32)),
                   p + "decay_shifts": torch.full((D, N), 15.0), p + "res_gate": torch.tensor([0.144])})
    sd.update(over)
    return sd


def _config(dims=DIMS, **ssm):
    return {"d_model": dims.d_model, "n_layer": dims.n_layer, "vocab_size": dims.vocab_size,
            "ssm_cfg": dict({"d_state": dims.d_state, "dt_rank": dims.dt_rank}, **ssm)}


def test_convert_state_dict_rules(tmp_path):
    """Each integer tensor equals its conversion rule computed independently in
    numpy (fp32 products, round half to even, clamps), the ternary matrices
    unpack to the quantized weights, and the converted model saves and loads."""
    rng = np.random.default_rng(0)
    sd = _state_dict(rng)
    # rounding ties and clamps of the decays
    sd["layers.0.base_decay_nums"][0, :4] = sd["layers.0.base_decay_nums"].new_tensor([16384.5, 16385.5, -3, 40000])
    p, logit_scale = ckpt.convert_state_dict({"_orig_mod." + k: v for k, v in sd.items()}, _config())
    n = {k: v.numpy() for k, v in sd.items()}
    assert np.array_equal(p.emb, np.clip(np.round(n["embedding.weight"] * 16), -127, 127).astype(np.int8))
    assert np.array_equal(p.gamma_f, np.round((n["norm_f.gamma"] * n["norm_f.step_size"]) * 256).astype(np.int16))
    ly = p.layers[0]
    assert ly.base[0, :4].tolist() == [16384, 16386, 0, 32000]
    assert np.array_equal(ly.base, np.clip(np.round(n["layers.0.base_decay_nums"]), 0, 32000).astype(np.int32))
    assert np.array_equal(ly.gamma, np.round(n["layers.0.norm.gamma"] * np.float32(0.75) * 256).astype(np.int16))
    assert np.array_equal(ly.conv_w, np.clip(np.round(n["layers.0.conv1d.weight"][:, 0] * 64), -127, 127))
    assert np.array_equal(ly.conv_b, np.round(n["layers.0.conv1d.bias"] * 1024).astype(np.int32))
    for key, attr, qin, qout in (("in_proj", "w_in", 4, 4), ("x_proj", "w_x", 4, 4), ("dt_proj", "w_dt", 4, 0)):
        w = n[f"layers.0.{key}.weight"]
        s = np.float32(np.abs(w).astype(np.float64).mean())
        wq = np.clip(np.round(w / s), -1, 1).astype(np.int8)
        assert np.array_equal(unpack_ternary(getattr(ly, attr), w.shape[1]), wq), key
        assert getattr(ly, {"w_in": "s_in", "w_x": "s_x", "w_dt": "s_dt"}[attr]) == \
            min(30, max(0, math.floor(qin - qout - math.log2(s) + 0.5)))
    s_out = float(np.abs(n["layers.0.out_proj.weight"]).mean())
    assert abs(ly.res_mult / 2.0 ** ly.res_shift - 16 * s_out * 0.144) < 1e-4 * 16 * s_out * 0.144
    assert (ly.k, ly.s_y) == (15, 14)
    s_head = float(np.abs(n["lm_head.weight"]).mean())
    assert abs(logit_scale - s_head / 16 / 8) < 1e-6 * logit_scale
    ckpt.save(p, str(tmp_path / "c.miq"), logit_scale)
    q, ls = ckpt.load(str(tmp_path / "c.miq"))
    _equal(p, q)
    assert ls == np.float32(logit_scale)


@pytest.mark.parametrize("change,needle", [
    ("drop", "no 'layers.1.x_proj.weight'"), ("shape", "shape"), ("extra", "does not use"),
    ("shifts", "uniform shift"), ("bias", "dt bias"), ("ssd", "no 'layers.0.x_proj.weight'|shape"),
])
def test_convert_rejects(change, needle):
    import torch
    rng = np.random.default_rng(1)
    sd = _state_dict(rng)
    cfg = _config()
    if change == "drop":
        del sd["layers.1.x_proj.weight"]
    elif change == "shape":
        sd["layers.0.in_proj.weight"] = sd["layers.0.in_proj.weight"][:, :32]
    elif change == "extra":
        sd["layers.0.mystery"] = torch.zeros(3)
    elif change == "shifts":
        sd["layers.1.decay_shifts"][0, 0] = 14.0
    elif change == "bias":
        sd["layers.0.dt_proj.bias"] = torch.full((DIMS.d_inner,), 0.5)
    elif change == "ssd":
        cfg = _config(use_ssd=True)
    with pytest.raises(ckpt.CheckpointError, match=needle):
        ckpt.convert_state_dict(sd, cfg)


def test_zero_dt_bias_is_accepted():
    import torch
    sd = _state_dict(np.random.default_rng(2))
    sd["layers.0.dt_proj.bias"] = torch.zeros(DIMS.d_inner)
    p, _ = ckpt.convert_state_dict(sd, _config())
    assert p.dims.n_layer == 2


def test_convert_reference_checkpoint_file(tmp_path):
    """A torch.save state dict on disk -> format-1 file (tensors only, loaded
    with weights_only=True), equal to the in-memory conversion."""
    import torch
    sd = _state_dict(np.random.default_rng(3))
    torch.save(sd, tmp_path / "ref.pt")
    p = ckpt.convert_reference_checkpoint(str(tmp_path / "ref.pt"), _config(), str(tmp_path / "out.miq"))
    q, _ = ckpt.load(str(tmp_path / "out.miq"))
    _equal(p, q)
    r, _ = ckpt.convert_state_dict(sd, _config())
    _equal(p, r)
    assert np.array_equal(pack_ternary(unpack_ternary(q.w_head, 64)), q.w_head)


# ------------------------------------------------ multi-head SSD block (V2)
SSD_DIMS = ModelDims(d_model=64, n_layer=2, vocab_size=90, d_state=16, dt_rank=0, block="ssd", n_heads=2,
                     d_head=32)


def _ssd_state_dict(rng, dims=SSD_DIMS):
    import torch
    d, D, N, H, V = dims.d_model, dims.d_inner, dims.d_state, dims.n_heads, dims.vocab_size
    f = lambda *s, sc=1.0: torch.from_numpy((rng.standard_normal(s) * sc).astype(np.float32))  # noqa: E731
    sd = {"embedding.weight": f(V, d), "norm_f.gamma": 1 + f(d, sc=0.1), "norm_f.step_size": torch.ones(1),
          "lm_head.weight": f(V, d, sc=d ** -1)}
    for i in range(dims.n_layer):
        p = f"layers.{i}."
        sd.update({p + "norm.gamma": 1 + f(d, sc=0.1), p + "norm.step_size": torch.tensor([1.25]),
                   p + "in_proj.weight": f(2 * D, d, sc=d ** -0.5), p + "conv1d.weight": f(D, 1, 4, sc=0.5),
                   p + "conv1d.bias": f(D, sc=0.1), p + "x_proj.weight": f(H * (1 + 2 * N), D, sc=D ** -0.5),
                   p + "A_log": torch.from_numpy(rng.uniform(-2.5, 0.0, H).astype(np.float32)),
                   p + "out_proj.weight": f(d, D, sc=D ** -0.5), p + "res_gate": torch.tensor([0.144])})
    return sd


def _ssd_config(dims=SSD_DIMS):
    return {"d_model": dims.d_model, "n_layer": dims.n_layer, "vocab_size": dims.vocab_size,
            "ssm_cfg": {"d_state": dims.d_state, "use_ssd": True, "n_heads": dims.n_heads, "d_head": dims.d_head}}


def test_ssd_round_trip_and_native_info(tmp_path):
    from mamba_int.native import NativeCheckpoint
    p = init_random_params(ModelDims(**SSD_DIMS.__dict__), 9)
    path = tmp_path / "v2.miq"
    ckpt.save(p, str(path), 0.5)
    q, _ = ckpt.load(str(path))
    _equal(p, q)
    i = NativeCheckpoint(str(path)).info
    assert (i.block, i.n_heads, i.d_head, i.d_state) == (1, 2, 32, 16)
    p.layers[1].decay_tab[0, 3] = 32769                      # outside [0, 2^15]
    ckpt.save(p, str(path), 0.5)
    with pytest.raises(ckpt.CheckpointError, match="decay numerator"):
        ckpt.load(str(path))
    st, msg = _native_open(path)
    assert st != 0 and "decay numerator" in msg


def test_convert_ssd_state_dict(tmp_path):
    """The V2 conversion: x_proj quantized over the reference's row order and
    reordered to planar [B | C | dt | 0]; A_log -> the decay table; V2 norm gain."""
    from mamba_int import ssd_decay_table
    sd = _ssd_state_dict(np.random.default_rng(4))
    p, _ = ckpt.convert_state_dict(sd, _ssd_config())
    assert p.dims.ssd and p.dims.xp_width == 80
    H, N, D = 2, 16, 64
    for i in range(2):
        ly = p.layers[i]
        w = sd[f"layers.{i}.x_proj.weight"].numpy()
        s = np.float32(np.abs(w).astype(np.float64).mean())
        wq = np.clip(np.round(w / s), -1, 1).astype(np.int8).reshape(H, 1 + 2 * N, D)
        got = unpack_ternary(ly.w_x, D)
        assert np.array_equal(got[:H * N], wq[:, 1:1 + N].reshape(-1, D))
        assert np.array_equal(got[H * N:2 * H * N], wq[:, 1 + N:].reshape(-1, D))
        assert np.array_equal(got[2 * H * N:2 * H * N + H], wq[:, 0])
        assert not got[2 * H * N + H:].any()
        assert np.array_equal(ly.decay_tab, ssd_decay_table(sd[f"layers.{i}.A_log"].numpy()))
        assert np.array_equal(ly.gamma, np.round(sd[f"layers.{i}.norm.gamma"].numpy() * np.float32(1.25) * 256))
        # out clamp +-100 (ssd_multihead.py:589-590) on out = acc * s / 16: |acc| <= floor(1600 / s)
        wo = sd[f"layers.{i}.out_proj.weight"].numpy()
        so = float(np.float32(np.abs(wo).astype(np.float64).mean()))
        assert ly.out_clamp == math.floor(1600 / so) and (ly.out_clamp + 1) * so / 16 > 100 >= ly.out_clamp * so / 16
    ckpt.save(p, str(tmp_path / "c.miq"), 1.0)
    _equal(p, ckpt.load(str(tmp_path / "c.miq"))[0])


def _as_format1(path):
    """Rewrites a format-2 file as the format-1 file of the same model under
    mi-spec-1 (out_clamp slots zero: the SSD block had no out_proj clamp)."""
    _rewrite(path, "layer_scalars",
             lambda raw: (np.frombuffer(raw, np.int32).reshape(-1, 8) * np.array([1] * 7 + [0], np.int32)).tobytes())
    b = bytearray(path.read_bytes())
    struct.pack_into("<I", b, 8, 1)
    b[16:32] = b"mi-spec-1".ljust(16, b"\0")
    path.write_bytes(bytes(b))


@pytest.mark.parametrize("ssd", [False, True])
def test_format1_files_are_read(tmp_path, ssd):
    """A format-1 (mi-spec-1) file loads in both readers; its SSD layers get
    out_clamp 0, the unclamped out_proj that spec computed."""
    from mamba_int.native import NativeCheckpoint
    p = init_random_params(ModelDims(**(SSD_DIMS if ssd else DIMS).__dict__), 9)
    path = tmp_path / "f1.miq"
    ckpt.save(p, str(path), 0.5)
    _as_format1(path)
    q, _ = ckpt.load(str(path))
    for ly in p.layers:
        ly.out_clamp = 0
    _equal(p, q)
    i = NativeCheckpoint(str(path)).info
    assert (i.format_version, i.spec) == (1, b"mi-spec-1")


@pytest.mark.parametrize("case,needle", [
    ("ssd_zero", "must be >= 1"), ("dyadic_nonzero", "has none"), ("format1_nonzero", "has none"),
    ("format1_spec2", "expected mi-spec-1"), ("format3", "format 3"),
])
def test_out_clamp_and_format_rules(tmp_path, case, needle):
    """Format-2 SSD layers carry an out clamp >= 1; dyadic layers and format-1
    files carry 0; the spec string matches the format."""
    ssd = case in ("ssd_zero", "format1_nonzero")
    p = init_random_params(ModelDims(**(SSD_DIMS if ssd else DIMS).__dict__), 9)
    path = tmp_path / "c.miq"
    ckpt.save(p, str(path), 0.5)
    put = lambda v: lambda raw: (np.frombuffer(raw, np.int32).reshape(-1, 8) * np.array([1] * 7 + [0], np.int32)
                                 + np.array([0] * 7 + [v], np.int32)).tobytes()  # noqa: E731
    if case == "ssd_zero":
        _rewrite(path, "layer_scalars", put(0))
    elif case == "dyadic_nonzero":
        _rewrite(path, "layer_scalars", put(500))
    elif case == "format1_nonzero":
        _as_format1(path)
        _rewrite(path, "layer_scalars", put(500))
    b = bytearray(path.read_bytes())
    if case == "format1_spec2":
        struct.pack_into("<I", b, 8, 1)
    elif case == "format3":
        struct.pack_into("<I", b, 8, 3)
    path.write_bytes(bytes(b))
    with pytest.raises(ckpt.CheckpointError, match=needle):
        ckpt.load(str(path))
    st, msg = _native_open(path)
    assert st != 0 and needle in msg, msg
