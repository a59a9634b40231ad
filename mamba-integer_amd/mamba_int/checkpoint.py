"""Integer checkpoints (format 2, spec mi-spec-2; format-1 files of spec
mi-spec-1 are read too) and the converter from the reference's float
checkpoints.

The reference exports inference weights as a bare 0xDAD1C stream
(``scripts/export_int8.py:50-135``) and reads them back with a loader that
stops after the conv taps (``src/cpp_engine/mamba_infer.cpp:46-118``).  An
integer checkpoint instead holds the integer parameters of ``ModelParams`` as a
table of named, typed, shaped tensors, each at a 256-byte aligned offset with
its CRC-32, so the native loader (``mi_checkpoint_open`` /
``mi_checkpoint_upload``) can validate it and copy it into one device buffer
with the kernels' alignment.  Layout (little-endian):

- header, 128 bytes: magic ``MIQCKPT\\0``, u32 format 2, u32 header bytes 128,
  char spec[16] ``mi-spec-2``, u32 d_model, n_layer, vocab_size, d_state,
  dt_rank, u32 tensor count, u64 table offset, u64 file bytes, f32
  logit_scale, u32 CRC-32 of the table, u32 block (0 dyadic scan, 1
  multi-head SSD), u32 n_heads, u32 d_head, zeros;
- table, 96 bytes per tensor: char name[48], u32 dtype (1 i8, 2 u8, 3 i16,
  4 i32, 5 f32), u32 ndim, u32 shape[4], u64 offset, u64 bytes, u32 CRC-32,
  u32 zero;
- the tensors: ``emb``, ``gamma_f``, ``w_head``, ``layer_scalars`` (int32
  [n_layer, 8]: s_in, s_x, s_dt, decay_shift, s_y, res_mult, res_shift,
  out_clamp; out_clamp is the SSD block's out_proj bound, >= 1, and 0 in
  dyadic-block layers and in every layer of a format-1 file) and
  per layer ``layers.{i}.{gamma, w_in, conv_w, conv_b, w_x, w_dt, base,
  w_out}`` (the SSD block: ``decay_tab`` in place of ``w_dt`` and ``base``).

``convert_state_dict`` maps a ``MambaIntegerModel`` float state dict (keys of
``mamba_integer_model.py:368-394,449-484``, ``ssd_multihead.py:481-522`` for
the multi-head SSD block, and ``rational_bitnet.py:150-158``) onto these
integers with the fixed-point formats of spec mi-spec-2 (sections 6 and 7 of
the spec list the rules).
"""
from __future__ import annotations

import math
import struct
import sys
import zlib
from typing import Dict, List, Mapping, Tuple

import numpy as np

from .params import (DECAY_MAX, DECAY_SHIFT, LayerParams, ModelDims, ModelParams, SSDLayerParams, out_clamp_for,
                     pack_ternary, ssd_decay_table)

MAGIC = b"MIQCKPT\0"
FORMAT = 2
SPEC = "mi-spec-2"
_SPEC_OF_FORMAT = {1: "mi-spec-1", 2: "mi-spec-2"}
ALIGN = 256
_HEADER = struct.Struct("<8sII16s5IIQQfIIII36x")
_ENTRY = struct.Struct("<48sII4IQQII")
_DTYPES = {1: np.int8, 2: np.uint8, 3: np.int16, 4: np.int32, 5: np.float32}
_CODES = {(np.dtype(v).kind, np.dtype(v).itemsize): k for k, v in _DTYPES.items()}
_LAYER_KEYS = ("gamma", "w_in", "conv_w", "conv_b", "w_x", "w_dt", "base", "w_out")
_SSD_KEYS = ("gamma", "w_in", "conv_w", "conv_b", "w_x", "decay_tab", "w_out")
BLOCK_DYADIC, BLOCK_SSD = 0, 1

assert _HEADER.size == 128 and _ENTRY.size == 96


class CheckpointError(ValueError):
    """A checkpoint file or state dict that does not satisfy the format."""


def _expected(dims: ModelDims) -> List[Tuple[str, np.dtype, Tuple[int, ...]]]:
    d, D, N, R, V = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank, dims.vocab_size
    out = [("emb", np.int8, (V, d)), ("gamma_f", np.int16, (d,)), ("w_head", np.uint8, (V, d // 4)),
           ("layer_scalars", np.int32, (dims.n_layer, 8))]
    shapes = {"gamma": (np.int16, (d,)), "w_in": (np.uint8, (2 * D, d // 4)), "conv_w": (np.int8, (D, 4)),
              "conv_b": (np.int32, (D,)), "w_x": (np.uint8, (dims.xp_width, D // 4)),
              "w_dt": (np.uint8, (D, R // 4)), "base": (np.int32, (D, N)), "w_out": (np.uint8, (d, D // 4)),
              "decay_tab": (np.int32, (dims.n_heads, 255))}
    for i in range(dims.n_layer):
        for k in (_SSD_KEYS if dims.ssd else _LAYER_KEYS):
            dt, sh = shapes[k]
            out.append((f"layers.{i}.{k}", dt, sh))
    return [(n, np.dtype(t), s) for n, t, s in out]


def _tensors(params: ModelParams) -> Dict[str, np.ndarray]:
    t = {"emb": params.emb, "gamma_f": params.gamma_f, "w_head": params.w_head}
    sc = np.zeros((params.dims.n_layer, 8), np.int32)
    ssd = params.dims.ssd
    for i, ly in enumerate(params.layers):
        sc[i] = (ly.s_in, ly.s_x, 0 if ssd else ly.s_dt, ly.k, ly.s_y, ly.res_mult, ly.res_shift,
                 ly.out_clamp if ssd else 0)
        if ssd and ly.out_clamp < 1:
            raise CheckpointError(f"layer {i}: out_clamp {ly.out_clamp} must be >= 1")
        for k in (_SSD_KEYS if ssd else _LAYER_KEYS):
            t[f"layers.{i}.{k}"] = getattr(ly, k)
    t["layer_scalars"] = sc
    return t


def save(params: ModelParams, path: str, logit_scale: float) -> None:
    """Writes ``params`` as a format-2 checkpoint; ``logit_scale`` (> 0) turns the
    int32 logits into the float logits of the drop-in model."""
    dims = params.dims
    dims.validate()
    if not logit_scale > 0:
        raise CheckpointError("logit_scale must be positive")
    have = _tensors(params)
    arrays = []
    for name, dt, shape in _expected(dims):
        a = np.ascontiguousarray(have[name])
        if a.dtype != dt or a.shape != shape:
            raise CheckpointError(f"{name}: {a.dtype}{a.shape}, the format wants {dt}{shape}")
        arrays.append((name, a.astype(dt.newbyteorder("<"), copy=False)))
    table_off = _HEADER.size
    off = -(-(table_off + _ENTRY.size * len(arrays)) // ALIGN) * ALIGN
    entries, blobs = [], []
    for name, a in arrays:
        raw = a.tobytes()
        shape = list(a.shape) + [0] * (4 - a.ndim)
        code = _CODES[(a.dtype.kind, a.dtype.itemsize)]
        entries.append(_ENTRY.pack(name.encode().ljust(48, b"\0"), code, a.ndim, *shape, off, len(raw),
                                   zlib.crc32(raw), 0))
        blobs.append((off, raw))
        off = -(-(off + len(raw)) // ALIGN) * ALIGN
    table = b"".join(entries)
    end = blobs[-1][0] + len(blobs[-1][1])
    header = _HEADER.pack(MAGIC, FORMAT, _HEADER.size, SPEC.encode().ljust(16, b"\0"), dims.d_model,
                          dims.n_layer, dims.vocab_size, dims.d_state, dims.dt_rank, len(arrays), table_off, end,
                          float(logit_scale), zlib.crc32(table), BLOCK_SSD if dims.ssd else BLOCK_DYADIC,
                          dims.n_heads if dims.ssd else 0, dims.d_head if dims.ssd else 0)
    buf = bytearray(end)
    buf[:len(header)] = header
    buf[table_off:table_off + len(table)] = table
    for o, raw in blobs:
        buf[o:o + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(buf)


def load(path: str) -> Tuple[ModelParams, float]:
    """Reads and validates a format-2 (or format-1) checkpoint (the checks of
    ``mi_checkpoint_open``); returns the integer parameters and logit_scale.  A
    format-1 file is an mi-spec-1 model: its SSD layers get out_clamp 0 (none)."""
    with open(path, "rb") as f:
        b = f.read()
    if len(b) < _HEADER.size:
        raise CheckpointError(f"{path}: shorter than the header")
    (magic, fmt, hbytes, spec, d_model, n_layer, vocab, d_state, dt_rank, nt, toff, fbytes, logit_scale,
     tcrc, block, n_heads, d_head) = _HEADER.unpack_from(b, 0)
    if magic != MAGIC:
        raise CheckpointError(f"{path}: not an integer checkpoint (bad magic)")
    if fmt not in _SPEC_OF_FORMAT or hbytes != _HEADER.size:
        raise CheckpointError(f"{path}: format {fmt} (this reader takes {sorted(_SPEC_OF_FORMAT)})")
    spec = spec.rstrip(b"\0").decode(errors="replace")
    if spec != _SPEC_OF_FORMAT[fmt]:
        raise CheckpointError(f"{path}: spec {spec!r} in a format-{fmt} file (expected {_SPEC_OF_FORMAT[fmt]})")
    if fbytes != len(b):
        raise CheckpointError(f"{path}: header says {fbytes} bytes, file has {len(b)}")
    if not logit_scale > 0:
        raise CheckpointError(f"{path}: logit_scale must be positive")
    if block not in (BLOCK_DYADIC, BLOCK_SSD):
        raise CheckpointError(f"{path}: block {block} unknown")
    if block == BLOCK_SSD:
        dims = ModelDims(d_model=d_model, n_layer=n_layer, vocab_size=vocab, d_state=d_state, dt_rank=dt_rank,
                         block="ssd", n_heads=n_heads, d_head=d_head)
    else:
        dims = ModelDims(d_model=d_model, n_layer=n_layer, vocab_size=vocab, d_state=d_state, dt_rank=dt_rank)
    try:
        dims.validate()
    except ValueError as e:
        raise CheckpointError(f"{path}: {e}") from None
    if toff < _HEADER.size or toff + nt * _ENTRY.size > len(b):
        raise CheckpointError(f"{path}: tensor table outside the file")
    table = b[toff:toff + nt * _ENTRY.size]
    if zlib.crc32(table) != tcrc:
        raise CheckpointError(f"{path}: tensor table CRC mismatch")
    found: Dict[str, np.ndarray] = {}
    for i in range(nt):
        name, code, ndim, s0, s1, s2, s3, off, nbytes, crc, _ = _ENTRY.unpack_from(table, i * _ENTRY.size)
        name = name.rstrip(b"\0").decode()
        if code not in _DTYPES or not 1 <= ndim <= 4:
            raise CheckpointError(f"{path}: tensor {name!r}: dtype {code} / ndim {ndim} invalid")
        shape = (s0, s1, s2, s3)[:ndim]
        dt = np.dtype(_DTYPES[code]).newbyteorder("<")
        if nbytes != math.prod(shape) * dt.itemsize:
            raise CheckpointError(f"{path}: tensor {name!r}: {nbytes} bytes for its shape")
        if off % ALIGN or off < toff + nt * _ENTRY.size or off + nbytes > len(b):
            raise CheckpointError(f"{path}: tensor {name!r}: misaligned or outside the file")
        raw = b[off:off + nbytes]
        if zlib.crc32(raw) != crc:
            raise CheckpointError(f"{path}: tensor {name!r}: CRC mismatch (corrupted data)")
        if name in found:
            raise CheckpointError(f"{path}: tensor {name!r} twice")
        found[name] = np.frombuffer(raw, dtype=dt).reshape(shape).astype(dt.newbyteorder("="))
    want = _expected(dims)
    for name, dt, shape in want:
        a = found.get(name)
        if a is None:
            raise CheckpointError(f"{path}: tensor {name!r} missing")
        if a.dtype != dt or a.shape != shape:
            raise CheckpointError(f"{path}: tensor {name!r}: dtype or shape does not match the dims")
        if dt == np.uint8 and np.any((a >> 1) & ~a & 0x55):
            raise CheckpointError(f"{path}: tensor {name!r} holds the invalid ternary code 0b10")
    if len(found) != len(want):
        raise CheckpointError(f"{path}: {len(found)} tensors, the format holds {len(want)}")
    sc = found["layer_scalars"]
    layers = []
    for i in range(n_layer):
        s_in, s_x, s_dt, k, s_y, res_mult, res_shift, out_clamp = (int(v) for v in sc[i])
        if (fmt == 1 or not dims.ssd) and out_clamp != 0:
            raise CheckpointError(f"{path}: layer {i}: out_clamp {out_clamp} where the format or block has none")
        if fmt == 2 and dims.ssd and out_clamp < 1:
            raise CheckpointError(f"{path}: layer {i}: out_clamp {out_clamp} must be >= 1")
        if not all(0 <= v <= 30 for v in (s_in, s_x, s_dt, s_y)) or not 0 <= res_shift <= 62:
            raise CheckpointError(f"{path}: layer {i}: a requant shift is outside its range")
        if k != DECAY_SHIFT:
            raise CheckpointError(f"{path}: layer {i}: decay shift {k} (the scan kernels take {DECAY_SHIFT})")
        g = lambda key: found[f"layers.{i}.{key}"]  # noqa: E731
        if dims.ssd:
            if g("decay_tab").min() < 0 or g("decay_tab").max() > 32768:
                raise CheckpointError(f"{path}: layer {i}: decay numerator outside [0,32768]")
            layers.append(SSDLayerParams(gamma=g("gamma"), w_in=g("w_in"), s_in=s_in, conv_w=g("conv_w"),
                                         conv_b=g("conv_b"), w_x=g("w_x"), s_x=s_x, decay_tab=g("decay_tab"),
                                         s_y=s_y, w_out=g("w_out"), res_mult=res_mult, res_shift=res_shift,
                                         out_clamp=out_clamp, k=k))
            continue
        if g("base").min(initial=0) < 0 or g("base").max(initial=0) > DECAY_MAX:
            raise CheckpointError(f"{path}: layer {i}: decay numerator outside [0,{DECAY_MAX}]")
        layers.append(LayerParams(gamma=g("gamma"), w_in=g("w_in"), s_in=s_in, conv_w=g("conv_w"),
                                  conv_b=g("conv_b"), w_x=g("w_x"), s_x=s_x, w_dt=g("w_dt"), s_dt=s_dt,
                                  base=g("base"), k=k, s_y=s_y, w_out=g("w_out"), res_mult=res_mult,
                                  res_shift=res_shift))
    return ModelParams(dims=dims, emb=found["emb"], layers=layers, gamma_f=found["gamma_f"],
                       w_head=found["w_head"]), float(logit_scale)


# ------------------------------------------------- float state dict -> integers
def _round_half_up(x: float) -> int:
    return int(math.floor(x + 0.5))


def _f32(t) -> "object":
    import torch
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float32)
    return torch.from_numpy(np.asarray(t, dtype=np.float32))


def ternary(w) -> Tuple[np.ndarray, float]:
    """weight_quant_ternary (``rational_bitnet.py:63-85``) in fp32 torch ops, as
    the reference computes it: s = max(mean|W|, 1e-6), Wq = clamp(round(W / s),
    -1, 1) (round half to even); returns (int8 Wq, float s)."""
    import torch
    w = _f32(w)
    s = torch.max(w.abs().mean(), torch.tensor(1e-6, dtype=torch.float32))
    q = torch.clamp(torch.round(w / s), -1, 1)
    return q.to(torch.int8).numpy(), float(s)


def _fixed(t, scale: float, lo: int, hi: int, dtype) -> np.ndarray:
    """round_half_even(t * scale) in fp32 (scale a power of two: exact), clamped."""
    import torch
    q = torch.round(_f32(t) * scale).to(torch.float64).clamp(lo, hi)
    return q.numpy().astype(dtype)


def requant_shift_for(w_scale: float, q_in: int, q_out: int) -> int:
    """Power-of-2 requant shift of an INT8 / DECAY_MOD BitLinear whose input is
    in Q(q_in) and output in Q(q_out): out ~ acc * w_scale * 2^(q_out - q_in),
    so s = round_half_up(q_in - q_out - log2(w_scale)), clamped to [0, 30]."""
    return min(30, max(0, _round_half_up(q_in - q_out - math.log2(w_scale))))


def residual_factor(w_scale: float, res_gate: float) -> Tuple[int, int]:
    """(res_mult, res_shift) of the out_proj epilogue: the float block adds
    out * res_gate (``mamba_integer_model.py:447``) with out = acc * w_scale / 16
    (Q4 input), i.e. 16 * w_scale * res_gate per unit of acc in the Q8
    residual; res_mult carries 15 significant bits."""
    f = 16.0 * w_scale * res_gate
    if f == 0.0:
        return 0, 0
    shift = min(62, max(0, 14 - math.floor(math.log2(abs(f)))))
    return _round_half_up(f * 2.0 ** shift), shift


def _strip(sd: Mapping[str, object]) -> Dict[str, object]:
    out = {}
    for k, v in sd.items():
        for p in ("_orig_mod.", "module."):
            if k.startswith(p):
                k = k[len(p):]
        out[k] = v
    return out


def convert_state_dict(state_dict: Mapping[str, object], config: dict,
                       strict: bool = True) -> Tuple[ModelParams, float]:
    """Integer parameters of a reference ``MambaIntegerModel`` (the dyadic-scan
    block, ``mamba_integer_model.py:368-394,466-484``, or with ``use_ssd`` the
    multi-head SSD block, ``ssd_multihead.py:471-522``) from its float state dict.

    Fixed-point formats of spec mi-spec-2: residual Q8, block activations Q4,
    conv taps Q6, conv bias Q10, gains Q8, decay_mod integer.  Hence
    emb = sat8(round(E * 16)); gamma = round(gamma * step_size * 256); ternary
    weights by weight_quant_ternary with the scale folded into a power-of-2
    shift (in_proj, x_proj: Q4 -> Q4; dt_proj: Q4 -> Q0) or into
    (res_mult, res_shift) with res_gate (out_proj); conv taps round(w * 64),
    bias round(b * 1024); decays clamp(round(base_decay_nums), 0, 32000) with
    the decay_shifts buffer (all 15); s_y = 14 (B, C in Q4: y in Q18 -> Q4);
    logit_scale = lm_head scale / 16 / sqrt(d_model) (the reference's
    output_scale, ``:483``); the SSD block's out_proj clamp to +-100
    (``ssd_multihead.py:589-590``) as the accumulator bound floor(1600 / s)
    of its out_proj weight scale s."""
    params, logit_scale, unused = convert_state_dict_keys(state_dict, config)
    if strict and unused:
        raise CheckpointError(f"state dict keys the integer model does not use: {unused[:5]}")
    return params, logit_scale


class _Reader:
    """Typed, shape-checked access to a stripped float state dict, recording the
    keys it reads."""

    def __init__(self, sd: Mapping[str, object], d_model: int):
        self.sd, self.d, self.used = sd, d_model, set()

    def get(self, key, shape):
        if key not in self.sd:
            raise CheckpointError(f"state dict has no {key!r}")
        t = _f32(self.sd[key])
        if tuple(t.shape) != tuple(shape):
            raise CheckpointError(f"{key}: shape {tuple(t.shape)}, config wants {tuple(shape)}")
        self.used.add(key)
        return t

    def gain(self, prefix):
        g = self.get(prefix + ".gamma", (self.d,)) * self.get(prefix + ".step_size", (1,))
        return _fixed(g, 256.0, -32767, 32767, np.int16)

    def unused(self):
        return sorted(k for k in self.sd if k not in self.used and not k.endswith("dt_proj.bias"))


def convert_state_dict_keys(state_dict: Mapping[str, object], config: dict) -> Tuple[ModelParams, float, List[str]]:
    """``convert_state_dict`` that returns the keys the integer model does not use
    (the ``unexpected_keys`` of ``load_state_dict(strict=False)``) instead of
    rejecting them.  A key it needs that is missing, or a value it cannot
    represent, still raises ``CheckpointError``."""
    sd = _strip(state_dict)
    dims = ModelDims.from_config(config)
    dims.validate()
    d, V = dims.d_model, dims.vocab_size
    rd = _Reader(sd, d)
    emb = _fixed(rd.get("embedding.weight", (V, d)), 16.0, -127, 127, np.int8)
    layers = [_convert_layer(f"layers.{i}.", dims, rd) for i in range(dims.n_layer)]
    w_head, s_head = ternary(rd.get("lm_head.weight", (V, d)))
    params = ModelParams(dims=dims, emb=emb, layers=layers, gamma_f=rd.gain("norm_f"), w_head=pack_ternary(w_head))
    return params, s_head / 16.0 / math.sqrt(d), rd.unused()


def convert_block_state_dict(state_dict: Mapping[str, object], config: dict):
    """One block's float state dict (the keys of ``MambaIntegerBlock``,
    ``mamba_integer_model.py:368-394``, or of ``MambaIntegerBlockV2`` with
    ``use_ssd``, ``ssd_multihead.py:481-522``, without a ``layers.{i}.``
    prefix) as (LayerParams or SSDLayerParams, unused keys)."""
    sd = _strip(state_dict)
    dims = ModelDims.from_config(config)
    dims.validate()
    rd = _Reader(sd, dims.d_model)
    return _convert_layer("", dims, rd), rd.unused()


def _convert_layer(p: str, dims: ModelDims, rd: "_Reader"):
    if dims.ssd:
        return _convert_ssd_layer(p, dims, rd.get, rd.gain)
    d, D, N, R = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank
    get = rd.get
    w_in, s_in_w = ternary(get(p + "in_proj.weight", (2 * D, d)))
    w_x, s_x_w = ternary(get(p + "x_proj.weight", (R + 2 * N, D)))
    w_dt, s_dt_w = ternary(get(p + "dt_proj.weight", (D, R)))
    w_out, s_out_w = ternary(get(p + "out_proj.weight", (d, D)))
    if p + "dt_proj.bias" in rd.sd:
        if float(get(p + "dt_proj.bias", (D,)).abs().max()) != 0.0:
            raise CheckpointError(f"{p}dt_proj.bias is non-zero: the integer block has no dt bias")
    shifts = get(p + "decay_shifts", (D, N))
    if float(shifts.min()) != float(shifts.max()) or float(shifts.min()) != DECAY_SHIFT:
        raise CheckpointError(f"{p}decay_shifts: the scan kernels take a uniform shift of {DECAY_SHIFT}")
    res_mult, res_shift = residual_factor(s_out_w, float(get(p + "res_gate", (1,))[0]))
    return LayerParams(
        gamma=rd.gain(p + "norm"),
        w_in=pack_ternary(w_in), s_in=requant_shift_for(s_in_w, 4, 4),
        conv_w=_fixed(get(p + "conv1d.weight", (D, 1, 4)).reshape(D, 4), 64.0, -127, 127, np.int8),
        conv_b=_fixed(get(p + "conv1d.bias", (D,)), 1024.0, -(2**31), 2**31 - 1, np.int32),
        w_x=pack_ternary(w_x), s_x=requant_shift_for(s_x_w, 4, 4),
        w_dt=pack_ternary(w_dt), s_dt=requant_shift_for(s_dt_w, 4, 0),
        base=_fixed(get(p + "base_decay_nums", (D, N)), 1.0, 0, DECAY_MAX, np.int32),
        k=DECAY_SHIFT, s_y=14,
        w_out=pack_ternary(w_out), res_mult=res_mult, res_shift=res_shift)


def _convert_ssd_layer(p: str, dims: ModelDims, get, gain) -> SSDLayerParams:
    """One MambaIntegerBlockV2 layer (``ssd_multihead.py:481-522``, spec section
    7): the x_proj rows, per head [dt, B (N), C (N)] (``:535-546``), are
    quantized with one scale over the whole matrix and then reordered to the
    planar [B | C | dt | zero padding] layout; A_log becomes the per-head decay
    table; the norm's eps is not part of the integer rule."""
    d, D, N, H = dims.d_model, dims.d_inner, dims.d_state, dims.n_heads
    w_in, s_in_w = ternary(get(p + "in_proj.weight", (2 * D, d)))
    wx, s_x_w = ternary(get(p + "x_proj.weight", (H * (1 + 2 * N), D)))
    wx = wx.reshape(H, 1 + 2 * N, D)
    planar = np.zeros((dims.xp_width, D), np.int8)
    planar[:H * N] = wx[:, 1:1 + N].reshape(H * N, D)
    planar[H * N:2 * H * N] = wx[:, 1 + N:].reshape(H * N, D)
    planar[2 * H * N:2 * H * N + H] = wx[:, 0]
    w_out, s_out_w = ternary(get(p + "out_proj.weight", (d, D)))
    res_mult, res_shift = residual_factor(s_out_w, float(get(p + "res_gate", (1,))[0]))
    return SSDLayerParams(
        gamma=gain(p + "norm"), w_in=pack_ternary(w_in), s_in=requant_shift_for(s_in_w, 4, 4),
        conv_w=_fixed(get(p + "conv1d.weight", (D, 1, 4)).reshape(D, 4), 64.0, -127, 127, np.int8),
        conv_b=_fixed(get(p + "conv1d.bias", (D,)), 1024.0, -(2**31), 2**31 - 1, np.int32),
        w_x=pack_ternary(planar), s_x=requant_shift_for(s_x_w, 4, 4),
        decay_tab=ssd_decay_table(get(p + "A_log", (H,)).numpy().astype(np.float64)), s_y=14,
        w_out=pack_ternary(w_out), res_mult=res_mult, res_shift=res_shift, out_clamp=out_clamp_for(s_out_w))


def convert_reference_checkpoint(state_dict_path: str, config: dict, out_path: str) -> ModelParams:
    """Loads a reference ``torch.save`` state dict (tensors only:
    ``weights_only=True``), converts it and writes a format-2 checkpoint."""
    import torch
    sd = torch.load(state_dict_path, map_location="cpu", weights_only=True)
    if isinstance(sd, dict) and "model" in sd and isinstance(sd["model"], dict):
        sd = sd["model"]
    params, logit_scale = convert_state_dict(sd, config)
    save(params, out_path, logit_scale)
    return params


def main(argv=None) -> int:
    """python -m mamba_int.checkpoint CONFIG.json STATE_DICT.pt OUT.miq"""
    import json
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 3:
        print(main.__doc__, file=sys.stderr)
        return 2
    with open(argv[0]) as f:
        config = json.load(f)
    p = convert_reference_checkpoint(argv[1], config, argv[2])
    print(f"wrote {argv[2]}: d_model={p.dims.d_model} n_layer={p.dims.n_layer} vocab={p.dims.vocab_size}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
