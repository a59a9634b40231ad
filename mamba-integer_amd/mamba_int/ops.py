"""Torch-facing wrappers of the C ABI (device tensors in, device tensors out).

PyTorch provides device memory and the current HIP stream; every op runs in
libmamba_int.so.  Inputs must be contiguous device tensors of the stated
dtype; outputs are allocated here (or passed in with ``out=``) so callers that
capture HIP graphs can keep static buffers.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import OUT_DECAY_MOD, OUT_FLOAT, OUT_INT8, OUT_INT32, OUT_RESIDUAL  # noqa: F401

_vp = ctypes.c_void_p


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else _vp(t.data_ptr())


def _stream():
    return _vp(torch.cuda.current_stream().cuda_stream)


def _req(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (libmamba_int has no host path)")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _opt(t, dtype, name):
    return None if t is None else _req(t, dtype, name)


# ------------------------------------------------------------------ scans
def dyadic_scan(x, b, c, decay_num, decay_shift: int = 15, h_in=None, h_out=None, out=None):
    """Config-1 scan: x int8 [B,L,D], b/c int8 [B,L,N], decay_num int32 [D,N] -> y int32 [B,L,D]."""
    _req(x, torch.int8, "x"); _req(b, torch.int8, "b"); _req(c, torch.int8, "c")
    _req(decay_num, torch.int32, "decay_num")
    B, L, D = x.shape
    N = b.shape[-1]
    y = out if out is not None else torch.empty((B, L, D), dtype=torch.int32, device=x.device)
    _req(y, torch.int32, "y")
    _lib.call("mi_dyadic_scan", _ptr(x), _ptr(b), _ptr(c), _ptr(decay_num), decay_shift, _ptr(y),
              _ptr(_opt(h_in, torch.int32, "h_in")), _ptr(_opt(h_out, torch.int32, "h_out")),
              B, L, D, N, _stream())
    return y


def dyadic_scan_f32(x, nums, shifts, scale_bits: int = 20):
    """Reference launch_dyadic_scan semantics: x fp32 [B,S,D], nums/shifts int32 -> h fp32."""
    _req(x, torch.float32, "x"); _req(nums, torch.int32, "nums"); _req(shifts, torch.int32, "shifts")
    B, S, D = x.shape
    h = torch.empty_like(x)
    _lib.call("mi_dyadic_scan_f32", _ptr(x), _ptr(nums), _ptr(shifts), _ptr(h), B, S, D, scale_bits, _stream())
    return h


def dyadic_scan_elementwise(u, nums, decay_shift: int, h_in=None, h_out=None):
    _req(u, torch.int32, "u"); _req(nums, torch.int32, "nums")
    B, L, C = u.shape
    h = torch.empty_like(u)
    _lib.call("mi_dyadic_scan_elementwise", _ptr(u), _ptr(nums), decay_shift, _ptr(h),
              _ptr(_opt(h_in, torch.int32, "h_in")), _ptr(_opt(h_out, torch.int32, "h_out")),
              B, L, C, _stream())
    return h


def dyadic_chunked_scan(u, nums, decay_shift: int, chunk: int, h_in=None, h_out=None):
    """Chunked elementwise recurrence (mi_dyadic_chunked_scan): u, nums int32
    [B,L,C] -> (h [B,L,C], final_h [B,nc,C], decay_to_end [B,nc,C] in Q30),
    nc = ceil(L / chunk)."""
    _req(u, torch.int32, "u"); _req(nums, torch.int32, "nums")
    if nums.shape != u.shape:
        raise ValueError(f"nums {tuple(nums.shape)} must match u {tuple(u.shape)}")
    if chunk < 1:
        raise ValueError(f"chunk={chunk} must be >= 1")
    B, L, C = u.shape
    nc = -(-L // chunk)
    h = torch.empty_like(u)
    final_h = torch.empty((B, nc, C), dtype=torch.int32, device=u.device)
    decay_to_end = torch.empty((B, nc, C), dtype=torch.int32, device=u.device)
    _lib.call("mi_dyadic_chunked_scan", _ptr(u), _ptr(nums), decay_shift, chunk, _ptr(h), _ptr(final_h),
              _ptr(decay_to_end), _ptr(_opt(h_in, torch.int32, "h_in")), _ptr(_opt(h_out, torch.int32, "h_out")),
              B, L, C, _stream())
    return h, final_h, decay_to_end


def ssd_chunked_scan(x, b, c, decay_num, decay_shift: int, chunk: int, chunk_states=None,
                     h_in=None, h_out=None):
    """Config-4 scan: x int8 [B,L,H,P], b/c int8 [B,L,H,N], decay_num int32 [H] -> y int32 [B,L,H,P]."""
    _req(x, torch.int8, "x"); _req(b, torch.int8, "b"); _req(c, torch.int8, "c")
    _req(decay_num, torch.int32, "decay_num")
    B, L, H, P = x.shape
    N = b.shape[-1]
    y = torch.empty((B, L, H, P), dtype=torch.int32, device=x.device)
    _lib.call("mi_ssd_chunked_scan", _ptr(x), _ptr(b), _ptr(c), _ptr(decay_num), decay_shift, _ptr(y),
              _ptr(_opt(chunk_states, torch.int32, "chunk_states")),
              _ptr(_opt(h_in, torch.int32, "h_in")), _ptr(_opt(h_out, torch.int32, "h_out")),
              B, L, H, P, N, chunk, _stream())
    return y


# ---------------------------------------------------------------- BitLinear
def pack_ternary(w: torch.Tensor) -> torch.Tensor:
    _req(w, torch.int8, "w")
    n, k = w.shape
    p = torch.empty((n, k // 4), dtype=torch.uint8, device=w.device)
    _lib.call("mi_pack_ternary", _ptr(w), _ptr(p), n, k, _stream())
    return p


def act_quant(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    _req(x, torch.float32, "x")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    _lib.call("mi_act_quant_f32", _ptr(x), _ptr(q), _ptr(s), m, k, _stream())
    return q, s


_OUT_DTYPE = {OUT_INT32: torch.int32, OUT_INT8: torch.int8, OUT_DECAY_MOD: torch.int8,
              OUT_RESIDUAL: torch.int32, OUT_FLOAT: torch.float32}
_ENTRY = {"auto": "mi_bitlinear", "gemm": "mi_bitlinear_gemm", "gemv": "mi_bitlinear_gemv"}


def bitlinear(a: torch.Tensor, w_packed: torch.Tensor, kind: int, n: int, k: Optional[int] = None,
              shift: int = 0, out: Optional[torch.Tensor] = None, res_mult: int = 0, res_shift: int = 0,
              x_scale: Optional[torch.Tensor] = None, w_scale: float = 0.0, path: str = "auto",
              lda: Optional[int] = None, m: Optional[int] = None,
              row_stats: Optional[torch.Tensor] = None, res_clamp: int = 0) -> torch.Tensor:
    """out = kind(a[:, :k] @ W^T).  a int8 [m, lda] (a row-strided view is passed by
    its storage with ``lda``); RESIDUAL updates ``out`` (int32 [m, n]) in place, its
    accumulator bounded to +-res_clamp first when res_clamp > 0."""
    if a.dtype != torch.int8 or not a.is_cuda:
        raise TypeError("a must be an int8 device tensor")
    if lda is None:
        _req(a, torch.int8, "a")
        lda = a.shape[-1]
    if m is None:
        m = a.shape[0]
    if k is None:
        k = lda
    _req(w_packed, torch.uint8, "w_packed")
    if out is None:
        if kind == OUT_RESIDUAL:
            raise ValueError("RESIDUAL output updates `out` in place; pass it")
        out = torch.empty((m, n), dtype=_OUT_DTYPE[kind], device=a.device)
    _req(out, _OUT_DTYPE[kind], "out")
    _lib.call(_ENTRY[path], _ptr(a), lda, _ptr(w_packed), _ptr(out), out.shape[-1], kind, m, n, k,
              shift, int(res_mult), res_shift, int(res_clamp), _ptr(_opt(x_scale, torch.float32, "x_scale")),
              ctypes.c_float(w_scale), _ptr(_opt(row_stats, torch.int64, "row_stats")), _stream())
    return out


# ---------------------------------------------------------------- block ops
def bitshift_norm(r: torch.Tensor, gamma: torch.Tensor, out=None, row_stats=None, v2: bool = False) -> torch.Tensor:
    """Integer BitShiftNorm of r int32 [T, d]; v2 selects BitShiftNormV2's table.  row_stats:
    full row sums int64 [T, 2], or per-block partials int64 [T, P, 2] (bitlinear_residual_parts)."""
    _req(r, torch.int32, "r"); _req(gamma, torch.int16, "gamma")
    T, d = r.shape
    o = out if out is not None else torch.empty((T, d), dtype=torch.int8, device=r.device)
    if row_stats is not None and row_stats.dim() == 3:
        _req(row_stats, torch.int64, "row_stats")
        if row_stats.shape[0] != T or row_stats.shape[2] != 2:
            raise ValueError(f"row_stats partials must be [{T}, P, 2], got {tuple(row_stats.shape)}")
        _lib.call("mi_bitshift_norm_parts", _ptr(r), _ptr(gamma), _ptr(o), T, d, _ptr(row_stats),
                  row_stats.shape[1], int(v2), _stream())
        return o
    _lib.call("mi_bitshift_norm_v2" if v2 else "mi_bitshift_norm", _ptr(r), _ptr(gamma), _ptr(o), T, d,
              _ptr(_opt(row_stats, torch.int64, "row_stats")), _stream())
    return o


def embed(ids: torch.Tensor, emb: torch.Tensor, out=None, row_stats=None) -> torch.Tensor:
    """r = emb[ids] << 4; with row_stats (int64 [layers, T, 2]) also the row
    statistics of r into layer 0 and zeros into the other layers."""
    _req(ids, torch.int64, "ids"); _req(emb, torch.int8, "emb")
    V, d = emb.shape
    T = ids.numel()
    r = out if out is not None else torch.empty((T, d), dtype=torch.int32, device=ids.device)
    layers = 0 if row_stats is None else row_stats.shape[0]
    _lib.call("mi_embed", _ptr(ids), _ptr(emb), _ptr(r), T, d, V,
              _ptr(_opt(row_stats, torch.int64, "row_stats")), layers, _stream())
    return r


def conv_squareplus(xz: torch.Tensor, d_inner: int, conv_w, conv_b, state_in=None, state_out=None,
                    out=None, batch: Optional[int] = None) -> torch.Tensor:
    """xz int8 [B, L, W] (or [B*L, W] with ``batch``), x branch = columns [0, d_inner)."""
    _req(xz, torch.int8, "xz"); _req(conv_w, torch.int8, "conv_w"); _req(conv_b, torch.int32, "conv_b")
    W = xz.shape[-1]
    B = xz.shape[0] if batch is None else batch
    L = xz.numel() // (W * B)
    xs = out if out is not None else torch.empty((B, L, d_inner), dtype=torch.int8, device=xz.device)
    _lib.call("mi_conv_squareplus", _ptr(xz), W, _ptr(conv_w), _ptr(conv_b),
              _ptr(_opt(state_in, torch.int8, "state_in")), _ptr(_opt(state_out, torch.int8, "state_out")),
              _ptr(xs), B, L, d_inner, _stream())
    return xs


def in_proj_conv(a: torch.Tensor, w_in: torch.Tensor, shift: int, d_inner: int, conv_w, conv_b, batch: int,
                 state_out: torch.Tensor, state_in=None, xs=None, xz=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Prefill in_proj + conv + squareplus: a int8 [batch*L, d_model] -> (xs int8 [batch*L, d_inner],
    xz int8 [batch*L, 2*d_inner] with only the z half written); state_out int8 [batch, 3, d_inner]
    receives the last three x rows of each sequence (state_in: the previous ones, or None for zeros)."""
    _req(a, torch.int8, "a"); _req(conv_w, torch.int8, "conv_w"); _req(conv_b, torch.int32, "conv_b")
    _req(state_out, torch.int8, "state_out")
    T, d = a.shape
    L = T // batch if batch else 0
    if batch and L * batch != T:
        raise ValueError("in_proj_conv: rows must be batch * len")
    if xs is None:
        xs = torch.empty((T, d_inner), dtype=torch.int8, device=a.device)
    if xz is None:
        xz = torch.empty((T, 2 * d_inner), dtype=torch.int8, device=a.device)
    _lib.call("mi_in_proj_conv", _ptr(a), a.stride(0), _ptr(w_in), shift, _ptr(conv_w), _ptr(conv_b),
              _ptr(_opt(state_in, torch.int8, "state_in")), _ptr(state_out), _ptr(xs), _ptr(xz), xz.stride(0),
              batch, L, d, d_inner, _stream())
    return xs, xz


def block_scan(xs, dm, xp, b_off: int, z, z_off: int, base, decay_shift: int, s_y: int,
               h_in=None, h_out=None, out=None, batch: Optional[int] = None) -> torch.Tensor:
    """Fused model scan; xs/dm int8 [B,L,D] (or [B*L,D] with ``batch``)."""
    for t, nm in ((xs, "xs"), (dm, "dm"), (xp, "xp"), (z, "z")):
        _req(t, torch.int8, nm)
    _req(base, torch.int32, "base")
    D, N = base.shape
    B = xs.shape[0] if batch is None else batch
    L = xs.numel() // (D * B)
    yo = out if out is not None else torch.empty((B, L, D), dtype=torch.int8, device=xs.device)
    _lib.call("mi_block_scan", _ptr(xs), _ptr(dm), _ptr(xp), xp.shape[-1], b_off, _ptr(z), z.shape[-1], z_off,
              _ptr(base), decay_shift, s_y, _ptr(yo), _ptr(_opt(h_in, torch.int32, "h_in")),
              _ptr(_opt(h_out, torch.int32, "h_out")), B, L, D, N, _stream())
    return yo


def ssd_block_scan(xs, xp, z, z_off: int, decay_tab, n_heads: int, d_state: int, s_y: int, h_in=None, h_out=None,
                   out=None, batch: Optional[int] = None) -> torch.Tensor:
    """Scan of the multi-head SSD block: xs int8 [B,L,D] (or [B*L,D] with ``batch``), xp int8
    planar [.., W], z int8 [.., Z] at column z_off, decay_tab int32 [H, 255] -> yo int8."""
    for t, nm in ((xs, "xs"), (xp, "xp"), (z, "z")):
        _req(t, torch.int8, nm)
    _req(decay_tab, torch.int32, "decay_tab")
    D = xs.shape[-1]
    B = xs.shape[0] if batch is None else batch
    L = xs.numel() // (D * B)
    yo = out if out is not None else torch.empty(xs.shape, dtype=torch.int8, device=xs.device)
    _lib.call("mi_ssd_block_scan", _ptr(xs), _ptr(xp), xp.shape[-1], _ptr(z), z.shape[-1], z_off, _ptr(decay_tab),
              n_heads, s_y, _ptr(yo), _ptr(_opt(h_in, torch.int32, "h_in")), _ptr(_opt(h_out, torch.int32, "h_out")),
              B, L, D, d_state, _stream())
    return yo


def argmax(logits: torch.Tensor, out=None) -> torch.Tensor:
    _req(logits, torch.int32, "logits")
    rows, cols = logits.shape
    o = out if out is not None else torch.empty((rows,), dtype=torch.int64, device=logits.device)
    _lib.call("mi_argmax_i32", _ptr(logits), cols, _ptr(o), rows, cols, _stream())
    return o


# ------------------------------------------------------ fused decode stages
def _stats(row_stats: Optional[torch.Tensor], m: int):
    """(pointer, parts) of a norm's row statistics: None, int64 [m, 2] (full
    sums) or int64 [m, parts, 2] (per-block partials, summed by the norm)."""
    if row_stats is None:
        return None, 1
    _req(row_stats, torch.int64, "row_stats")
    if row_stats.dim() == 2:
        row_stats = row_stats.unsqueeze(1)
    if row_stats.dim() != 3 or row_stats.shape[0] != m or row_stats.shape[2] != 2:
        raise ValueError(f"row_stats must be [{m}, 2] or [{m}, parts, 2], got {tuple(row_stats.shape)}")
    return _ptr(row_stats), row_stats.shape[1]


def bitlinear_residual_parts(a: torch.Tensor, w_packed: torch.Tensor, r: torch.Tensor, res_mult: int,
                             res_shift: int, stats_parts: torch.Tensor, res_clamp: int = 0) -> None:
    """Decode out_proj: r (int32 [m, n], m <= 64) += rescaled a @ W^T (accumulator bounded to
    +-res_clamp first when res_clamp > 0), and stats_parts (int64 [m, ceil(n/16), 2]) <- the
    per-16-feature (sum, sum of squares) of the new rows."""
    _req(a, torch.int8, "a"); _req(w_packed, torch.uint8, "w_packed"); _req(r, torch.int32, "r")
    _req(stats_parts, torch.int64, "stats_parts")
    m, n = r.shape
    k = a.shape[-1]
    if a.shape[0] != m or tuple(stats_parts.shape) != (m, (n + 15) // 16, 2):
        raise ValueError(f"a must be [{m}, k] and stats_parts [{m}, {(n + 15) // 16}, 2]")
    _lib.call("mi_bitlinear_residual_parts", _ptr(a), k, _ptr(w_packed), _ptr(r), n, m, n, k, int(res_mult),
              res_shift, int(res_clamp), _ptr(stats_parts), _stream())


def norm_bitlinear(r: torch.Tensor, gamma: torch.Tensor, w_packed: torch.Tensor, kind: int, n: int,
                   shift: int = 0, out=None, row_stats=None) -> torch.Tensor:
    """BitShiftNorm of r (int32 [m, k], m <= 64) fused into the BitLinear GEMV (INT8 or INT32 out)."""
    _req(r, torch.int32, "r"); _req(gamma, torch.int16, "gamma"); _req(w_packed, torch.uint8, "w_packed")
    m, k = r.shape
    o = out if out is not None else torch.empty((m, n), dtype=_OUT_DTYPE[kind], device=r.device)
    _req(o, _OUT_DTYPE[kind], "out")
    sp, parts = _stats(row_stats, m)
    _lib.call("mi_norm_bitlinear", _ptr(r), sp, parts, _ptr(gamma), _ptr(w_packed), _ptr(o), o.shape[-1], kind,
              m, n, k, shift, _stream())
    return o


def norm_in_proj_conv(r, gamma, w_in, s_in: int, conv_w, conv_b, conv_state, xs, xz, row_stats=None,
                      w_x=None, xpart=None, v2: bool = False) -> None:
    """Decode stage: norm + in_proj GEMV + conv step + squareplus (x half -> xs, conv_state
    updated in place), z half -> xz[:, d_inner:].  With w_x and xpart [m, d_inner/16, nx]
    int32, also the per-16-channel x_proj partials; v2: BitShiftNormV2's table."""
    _req(r, torch.int32, "r"); _req(gamma, torch.int16, "gamma"); _req(w_in, torch.uint8, "w_in")
    _req(conv_w, torch.int8, "conv_w"); _req(conv_b, torch.int32, "conv_b")
    _req(conv_state, torch.int8, "conv_state"); _req(xs, torch.int8, "xs"); _req(xz, torch.int8, "xz")
    m, d = r.shape
    D = conv_w.shape[0]
    stats, parts = _stats(row_stats, m)
    if v2 and xpart is not None:
        raise ValueError("the V2 norm stage has no x_proj partials")
    if xpart is None:
        _lib.call("mi_norm_v2_in_proj_conv" if v2 else "mi_norm_in_proj_conv", _ptr(r), stats, parts, _ptr(gamma),
                  _ptr(w_in), s_in, _ptr(conv_w),
                  _ptr(conv_b), _ptr(conv_state), _ptr(xs), _ptr(xz), m, d, D, _stream())
        return
    _req(xpart, torch.int32, "xpart"); _req(w_x, torch.uint8, "w_x")
    if tuple(xpart.shape[:2]) != (m, D // 16):
        raise ValueError(f"xpart must be [m, d_inner/16, nx], got {tuple(xpart.shape)}")
    _lib.call("mi_norm_in_proj_conv_xpart", _ptr(r), stats, parts, _ptr(gamma), _ptr(w_in), s_in, _ptr(conv_w),
              _ptr(conv_b), _ptr(conv_state), _ptr(xs), _ptr(xz), _ptr(w_x), xpart.shape[-1], _ptr(xpart), m, d, D,
              _stream())


def conv_step_xproj(xz, d_inner: int, conv_w, conv_b, conv_state, w_x, s_x: int, nx: int, xs=None, xp=None):
    """Decode stage: conv step + squareplus of the x half of xz (int8 [m, >= d_inner]) with
    the conv state updated in place -> xs, then x_proj (INT8, shift s_x) -> xp int8 [m, >= nx]."""
    _req(xz, torch.int8, "xz"); _req(conv_w, torch.int8, "conv_w"); _req(conv_b, torch.int32, "conv_b")
    _req(conv_state, torch.int8, "conv_state"); _req(w_x, torch.uint8, "w_x")
    m = xz.shape[0]
    if xs is None:
        xs = torch.empty((m, d_inner), dtype=torch.int8, device=xz.device)
    if xp is None:
        xp = torch.empty((m, nx), dtype=torch.int8, device=xz.device)
    _req(xs, torch.int8, "xs"); _req(xp, torch.int8, "xp")
    if tuple(xs.shape) != (m, d_inner) or xp.shape[0] != m or xp.shape[-1] < nx:
        raise ValueError(f"xs must be [{m}, {d_inner}] and xp [{m}, >= {nx}]")
    _lib.call("mi_conv_step_xproj", _ptr(xz), xz.shape[-1], _ptr(conv_w), _ptr(conv_b), _ptr(conv_state), _ptr(xs),
              _ptr(w_x), s_x, nx, _ptr(xp), xp.shape[-1], m, d_inner, _stream())
    return xs, xp


def conv_step_xpart(xz, d_inner: int, conv_w, conv_b, conv_state, w_x, nx: int, xs=None, xpart=None):
    """Decode stage: conv step + squareplus of the x half of xz (int8 [m, >= d_inner]) with
    the conv state updated in place -> xs, and the exact int32 x_proj sums over the four
    channel quarters -> xpart [m, 4, nx] (finished by xpart_dt_scan_step)."""
    _req(xz, torch.int8, "xz"); _req(conv_w, torch.int8, "conv_w"); _req(conv_b, torch.int32, "conv_b")
    _req(conv_state, torch.int8, "conv_state"); _req(w_x, torch.uint8, "w_x")
    m = xz.shape[0]
    if xs is None:
        xs = torch.empty((m, d_inner), dtype=torch.int8, device=xz.device)
    if xpart is None:
        xpart = torch.empty((m, 4, nx), dtype=torch.int32, device=xz.device)
    _req(xs, torch.int8, "xs"); _req(xpart, torch.int32, "xpart")
    if tuple(xs.shape) != (m, d_inner) or tuple(xpart.shape) != (m, 4, nx):
        raise ValueError(f"xs must be [{m}, {d_inner}] and xpart [{m}, 4, {nx}]")
    _lib.call("mi_conv_step_xpart", _ptr(xz), xz.shape[-1], _ptr(conv_w), _ptr(conv_b), _ptr(conv_state), _ptr(xs),
              _ptr(w_x), nx, _ptr(xpart), m, d_inner, _stream())
    return xs, xpart


def xpart_dt_scan_step(xpart, s_x: int, dt_rank: int, w_dt, s_dt: int, xs, z, z_off: int, base,
                       decay_shift: int, s_y: int, h_state, yo) -> None:
    """Decode stage: x_proj from per-block partials + dt_proj + decay + dt + scan step + gate -> yo."""
    for t, nm in ((xs, "xs"), (z, "z"), (yo, "yo")):
        _req(t, torch.int8, nm)
    _req(xpart, torch.int32, "xpart"); _req(w_dt, torch.uint8, "w_dt")
    _req(base, torch.int32, "base"); _req(h_state, torch.int32, "h_state")
    m = xs.shape[0]
    D, N = base.shape
    if xpart.shape[0] != m or xpart.shape[-1] != dt_rank + 2 * N:
        raise ValueError(f"xpart must be [m, nblk, dt_rank + 2*d_state], got {tuple(xpart.shape)}")
    _lib.call("mi_xpart_dt_scan_step", _ptr(xpart), xpart.shape[1], s_x, dt_rank, _ptr(w_dt), s_dt, _ptr(xs),
              _ptr(z), z.shape[-1], z_off, _ptr(base), decay_shift, s_y, _ptr(h_state), _ptr(yo), m, D, N,
              _stream())


def dt_scan_step(xp, dt_rank: int, w_dt, s_dt: int, xs, z, z_off: int, base, decay_shift: int, s_y: int,
                 h_state, yo) -> None:
    """Decode stage: dt_proj + decay + dt + scan state update + y + gate + requant -> yo."""
    for t, nm in ((xp, "xp"), (xs, "xs"), (z, "z"), (yo, "yo")):
        _req(t, torch.int8, nm)
    _req(w_dt, torch.uint8, "w_dt"); _req(base, torch.int32, "base"); _req(h_state, torch.int32, "h_state")
    m = xs.shape[0]
    D, N = base.shape
    _lib.call("mi_dt_scan_step", _ptr(xp), xp.shape[-1], dt_rank, _ptr(w_dt), s_dt, _ptr(xs), _ptr(z),
              z.shape[-1], z_off, _ptr(base), decay_shift, s_y, _ptr(h_state), _ptr(yo), m, D, N, _stream())


def xproj_dt_scan_step(xs, w_x, s_x: int, dt_rank: int, w_dt, s_dt: int, z, z_off: int, base,
                       decay_shift: int, s_y: int, h_state, yo) -> None:
    """Decode stage: x_proj + dt_proj + decay + dt + scan state update + y + gate + requant."""
    for t, nm in ((xs, "xs"), (z, "z"), (yo, "yo")):
        _req(t, torch.int8, nm)
    _req(w_x, torch.uint8, "w_x"); _req(w_dt, torch.uint8, "w_dt")
    _req(base, torch.int32, "base"); _req(h_state, torch.int32, "h_state")
    m = xs.shape[0]
    D, N = base.shape
    _lib.call("mi_xproj_dt_scan_step", _ptr(xs), _ptr(w_x), s_x, dt_rank, _ptr(w_dt), s_dt, _ptr(z),
              z.shape[-1], z_off, _ptr(base), decay_shift, s_y, _ptr(h_state), _ptr(yo), m, D, N, _stream())


def norm_bitlinear_argmax(r, gamma, w_packed, n: int, keys, logits=None, row_stats=None) -> None:
    """lm_head (norm + INT32 GEMV) writing per-64-output partial argmax keys [m, ceil(n/64)]
    and, when given, the logits."""
    _req(r, torch.int32, "r"); _req(gamma, torch.int16, "gamma"); _req(w_packed, torch.uint8, "w_packed")
    _req(keys, torch.int64, "keys")
    m, k = r.shape
    if tuple(keys.shape) != (m, (n + 63) // 64):
        raise ValueError(f"keys must be [{m}, {(n + 63) // 64}], got {tuple(keys.shape)}")
    ldo = 0
    if logits is not None:
        _req(logits, torch.int32, "logits")
        ldo = logits.stride(0)
    sp, parts = _stats(row_stats, m)
    _lib.call("mi_norm_bitlinear_argmax", _ptr(r), sp, parts, _ptr(gamma), _ptr(w_packed),
              _ptr(logits) if logits is not None else None, ldo, _ptr(keys), m, n, k, _stream())


def argmax_keys(keys, out=None) -> torch.Tensor:
    """ids [rows] int64 from the partial keys of norm_bitlinear_argmax."""
    _req(keys, torch.int64, "keys")
    rows, nk = keys.shape
    out = torch.empty((rows,), dtype=torch.int64, device=keys.device) if out is None else out
    _req(out, torch.int64, "out")
    _lib.call("mi_argmax_keys", _ptr(keys), nk, _ptr(out), rows, _stream())
    return out


def embed_argmax(keys, ids_out, emb, r, row_stats) -> None:
    """Greedy pick from partial keys, then the embedding (with row statistics) of the picks."""
    _req(keys, torch.int64, "keys"); _req(ids_out, torch.int64, "ids_out"); _req(emb, torch.int8, "emb")
    _req(r, torch.int32, "r"); _req(row_stats, torch.int64, "row_stats")
    T, nk = keys.shape
    V, d = emb.shape
    _lib.call("mi_embed_argmax", _ptr(keys), nk, _ptr(ids_out), _ptr(emb), _ptr(r), T, d, V, _ptr(row_stats),
              row_stats.shape[0], _stream())
