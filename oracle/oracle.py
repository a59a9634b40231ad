"""Python face of the CPU oracle (``mi_oracle.c``) — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the test oracle or the timed CPU baseline.
The product package never imports it.

Each wrapper takes and returns numpy arrays; ``OracleModel`` orchestrates the
per-op calls in the block order of ``MambaIntegerBlock.forward``
(``mamba_integer_model.py:396-447``) and ``MambaIntegerModel.forward``
(``:486-495``), plus the recurrent decode step the reference lacks
(``scripts/inference.py:147-161`` recomputes the whole prefix instead).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_REPO = os.path.dirname(_HERE)
_PKG_DIR = os.path.join(_REPO, "mamba-integer_amd")
if _PKG_DIR not in sys.path:
    sys.path.insert(0, _PKG_DIR)

from mamba_int.params import ModelParams  # noqa: E402

OUT_INT32, OUT_INT8, OUT_DECAY_MOD, OUT_RESIDUAL, OUT_FLOAT = 0, 1, 2, 3, 4

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        src = os.path.join(_HERE, "mi_oracle.c")
        if (not os.path.exists(_LIB_PATH)
                or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src)):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.mo_version.restype = ctypes.c_char_p
        L.mo_set_threads.argtypes = [I]
        L.mo_set_mutation.argtypes = [I]
        L.mo_isqrt.argtypes = [ctypes.c_uint64]
        L.mo_isqrt.restype = ctypes.c_uint64
        L.mo_dyadic_scan.argtypes = [P, P, P, P, I, P, P, I, I, I, I]
        L.mo_dyadic_scan_f32.argtypes = [P, P, P, P, I, I, I, I]
        L.mo_dyadic_scan_elementwise.argtypes = [P, P, I, P, P, I, I, I]
        L.mo_ssd_chunked_scan.argtypes = [P, P, P, P, I, P, P, P, I, I, I, I, I, I]
        L.mo_dyadic_chunked_scan.argtypes = [P, P, I, I, P, P, P, P, I, I, I]
        L.mo_pack_ternary.argtypes = [P, P, I, I]
        L.mo_unpack_ternary.argtypes = [P, P, I, I]
        L.mo_bitlinear.argtypes = [P, P, P, I, I, I, I, I, ctypes.c_int32, I, ctypes.c_int32, P, ctypes.c_float]
        L.mo_bitlinear_unpacked.argtypes = [P, P, P, I, I, I, I, I, ctypes.c_int32, I, ctypes.c_int32, P,
                                            ctypes.c_float]
        L.mo_act_quant_f32.argtypes = [P, P, P, I, I]
        L.mo_bitshift_norm.argtypes = [P, P, P, I, I]
        L.mo_squareplus_q.argtypes = [ctypes.c_int32]
        L.mo_squareplus_q.restype = ctypes.c_int8
        L.mo_conv_squareplus.argtypes = [P, I, P, P, P, P, I, I, I]
        L.mo_dt_q16.argtypes = [I]
        L.mo_dt_q16.restype = ctypes.c_int32
        L.mo_gate_q15.argtypes = [I]
        L.mo_gate_q15.restype = ctypes.c_int32
        L.mo_block_scan.argtypes = [P, P, P, I, I, P, I, I, P, I, I, P, P, I, I, I, I]
        L.mo_embed.argtypes = [P, P, P, I, I]
        L.mo_bitshift_norm_v2.argtypes = [P, P, P, I, I]
        L.mo_unit_q7.argtypes = [P, P, I]
        L.mo_ssd_v2_scan.argtypes = [P, P, I, P, I, I, P, I, P, P, I, I, I, I, I]
        L.mo_set_threads(len(os.sched_getaffinity(0)))
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def set_threads(n: int) -> None:
    lib().mo_set_threads(int(n))


def set_mutation(m: int) -> None:
    lib().mo_set_mutation(int(m))


def version() -> str:
    return lib().mo_version().decode()


# ------------------------------------------------------------------ scans
def dyadic_scan(x, Bm, Cm, ndec, k, h_state=None):
    x, Bm, Cm, ndec = _c(x, np.int8), _c(Bm, np.int8), _c(Cm, np.int8), _c(ndec, np.int32)
    B, L, D = x.shape
    N = Bm.shape[-1]
    y = np.empty((B, L, D), np.int32)
    hs = None if h_state is None else _c(h_state, np.int32).copy()
    rc = lib().mo_dyadic_scan(_p(x), _p(Bm), _p(Cm), _p(ndec), k, _p(y), _p(hs), B, L, D, N)
    if rc:
        raise ValueError("oracle dyadic_scan rejected its arguments")
    return (y, hs) if h_state is not None else y


def dyadic_scan_f32(x, nums, shifts, scale_bits=20):
    x, nums, shifts = _c(x, np.float32), _c(nums, np.int32), _c(shifts, np.int32)
    B, S, D = x.shape
    h = np.empty_like(x)
    lib().mo_dyadic_scan_f32(_p(x), _p(nums), _p(shifts), _p(h), B, S, D, scale_bits)
    return h


def dyadic_scan_elementwise(u, n, k, h_state=None):
    u, n = _c(u, np.int32), _c(n, np.int32)
    B, L, C = u.shape
    h = np.empty_like(u)
    hs = None if h_state is None else _c(h_state, np.int32).copy()
    lib().mo_dyadic_scan_elementwise(_p(u), _p(n), k, _p(h), _p(hs), B, L, C)
    return (h, hs) if h_state is not None else h


def dyadic_chunked_scan(u, n, k, chunk, h_state=None):
    """Chunked elementwise scan (the outputs of ssd_chunked_scan_forward): u, n
    int32 [B,L,C] -> h [B,L,C], final_h [B,nc,C], decay_to_end [B,nc,C] (Q30),
    and the final state when h_state is given."""
    u, n = _c(u, np.int32), _c(n, np.int32)
    B, L, C = u.shape
    nc = -(-L // chunk)
    h = np.empty_like(u)
    fh = np.empty((B, nc, C), np.int32)
    dte = np.empty((B, nc, C), np.int32)
    hs = None if h_state is None else _c(h_state, np.int32).copy()
    lib().mo_dyadic_chunked_scan(_p(u), _p(n), k, chunk, _p(h), _p(fh), _p(dte), _p(hs), B, L, C)
    return (h, fh, dte, hs) if h_state is not None else (h, fh, dte)


def ssd_chunked_scan(x, Bm, Cm, ndec, k, chunk, want_chunk_states=False, h_state=None):
    x, Bm, Cm, ndec = _c(x, np.int8), _c(Bm, np.int8), _c(Cm, np.int8), _c(ndec, np.int32)
    B, L, H, P = x.shape
    N = Bm.shape[-1]
    nc = -(-L // chunk)
    y = np.empty((B, L, H, P), np.int32)
    cst = np.empty((B, nc, H, P, N), np.int32) if want_chunk_states else None
    hs = None if h_state is None else _c(h_state, np.int32).copy()
    rc = lib().mo_ssd_chunked_scan(_p(x), _p(Bm), _p(Cm), _p(ndec), k, _p(y), _p(cst), _p(hs),
                                   B, L, H, P, N, chunk)
    if rc:
        raise ValueError("oracle ssd_chunked_scan rejected its arguments")
    out = [y]
    if want_chunk_states:
        out.append(cst)
    if h_state is not None:
        out.append(hs)
    return out[0] if len(out) == 1 else tuple(out)


# ---------------------------------------------------------------- ternary
def pack_ternary(w):
    w = _c(w, np.int8)
    N, K = w.shape
    p = np.empty((N, K // 4), np.uint8)
    if lib().mo_pack_ternary(_p(w), _p(p), N, K):
        raise ValueError("ternary weights must lie in {-1,0,1}")
    return p


def unpack_ternary(p, K):
    p = _c(p, np.uint8)
    N = p.shape[0]
    w = np.empty((N, K), np.int8)
    lib().mo_unpack_ternary(_p(p), _p(w), N, K)
    return w


def bitlinear(a, wp, kind, shift=0, residual=None, res_mult=0, res_shift=0,
              x_scale=None, w_scale=0.0, res_clamp=0):
    """BitLinear of int8 rows a [M,K] against packed ternary wp [N,K/4], or
    against weights already unpacked to int8 [N,K] (same result).  res_clamp > 0
    bounds the RESIDUAL accumulator to +-res_clamp first (spec rule 7.9)."""
    a = _c(a, np.int8)
    unpacked = wp.dtype == np.int8
    wp = _c(wp, np.int8 if unpacked else np.uint8)
    M, K = a.shape
    N = wp.shape[0]
    if kind == OUT_INT32:
        out = np.empty((M, N), np.int32)
    elif kind in (OUT_INT8, OUT_DECAY_MOD):
        out = np.empty((M, N), np.int8)
    elif kind == OUT_RESIDUAL:
        out = _c(residual, np.int32).copy()
    else:
        out = np.empty((M, N), np.float32)
    xs = None if x_scale is None else _c(x_scale, np.float32)
    fn = lib().mo_bitlinear_unpacked if unpacked else lib().mo_bitlinear
    fn(_p(a), _p(wp), _p(out), kind, M, N, K, shift, int(res_mult), res_shift, int(res_clamp), _p(xs),
       ctypes.c_float(w_scale))
    return out


def act_quant_f32(x):
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().mo_act_quant_f32(_p(x), _p(q), _p(s), M, K)
    return q, s


# -------------------------------------------------------------- block ops
def bitshift_norm(r, gamma):
    r, gamma = _c(r, np.int32), _c(gamma, np.int16)
    T, d = r.shape
    out = np.empty((T, d), np.int8)
    lib().mo_bitshift_norm(_p(r), _p(gamma), _p(out), T, d)
    return out


def bitshift_norm_v2(r, gamma):
    """BitShiftNormV2 (spec rule 7.1)."""
    r, gamma = _c(r, np.int32), _c(gamma, np.int16)
    T, d = r.shape
    out = np.empty((T, d), np.int8)
    lib().mo_bitshift_norm_v2(_p(r), _p(gamma), _p(out), T, d)
    return out


def unit_q7(v):
    """Unit vector in Q7 of an int8 vector (spec rule 7.4)."""
    v = _c(v, np.int8).reshape(-1)
    out = np.empty_like(v)
    lib().mo_unit_q7(_p(v), _p(out), v.size)
    return out


def ssd_v2_scan(xs, xp, z_src, z_off, tab, s_y, n_heads, d_state, h_state=None):
    """SSD block scan (spec rules 7.3-7.8): xs [B,L,D], xp [B,L,W] planar,
    z_src [B,L,Z]; tab int32 [H,255]; returns yo [B,L,D] and the state [B,D,N]."""
    xs, xp, z_src, tab = _c(xs, np.int8), _c(xp, np.int8), _c(z_src, np.int8), _c(tab, np.int32)
    B, L, D = xs.shape
    H = n_heads
    P = D // H
    W = xp.shape[-1]
    N = d_state
    hs = np.zeros((B, D, N), np.int32) if h_state is None else _c(h_state, np.int32).copy()
    yo = np.empty((B, L, D), np.int8)
    lib().mo_ssd_v2_scan(_p(xs), _p(xp), W, _p(z_src), z_src.shape[-1], z_off, _p(tab), s_y, _p(yo), _p(hs),
                         B, L, H, P, N)
    return yo, hs


def squareplus_q(c: int) -> int:
    return int(lib().mo_squareplus_q(int(c)))


def dt_q16(dm: int) -> int:
    return int(lib().mo_dt_q16(int(dm)))


def gate_q15(z: int) -> int:
    return int(lib().mo_gate_q15(int(z)))


def conv_squareplus(xz, D, conv_w, conv_b, state=None):
    """xz int8 [B,L,W] (x branch = columns [0,D)); returns xs [B,L,D] and the new state."""
    xz = _c(xz, np.int8)
    B, L, W = xz.shape
    st = np.zeros((B, 3, D), np.int8) if state is None else _c(state, np.int8).copy()
    xs = np.empty((B, L, D), np.int8)
    lib().mo_conv_squareplus(_p(xz), W, _p(_c(conv_w, np.int8)), _p(_c(conv_b, np.int32)),
                             _p(st), _p(xs), B, L, D)
    return xs, st


def block_scan(xs, dm, xp, b_off, z_src, z_off, base, k, s_y, h_state=None):
    xs, dm, xp, z_src = _c(xs, np.int8), _c(dm, np.int8), _c(xp, np.int8), _c(z_src, np.int8)
    base = _c(base, np.int32)
    B, L, D = xs.shape
    N = base.shape[1]
    hs = np.zeros((B, D, N), np.int32) if h_state is None else _c(h_state, np.int32).copy()
    yo = np.empty((B, L, D), np.int8)
    lib().mo_block_scan(_p(xs), _p(dm), _p(xp), xp.shape[-1], b_off, _p(z_src), z_src.shape[-1],
                        z_off, _p(base), k, s_y, _p(yo), _p(hs), B, L, D, N)
    return yo, hs


def embed(ids, emb):
    ids = _c(ids, np.int64)
    emb = _c(emb, np.int8)
    T = ids.size
    d = emb.shape[1]
    r = np.empty((T, d), np.int32)
    lib().mo_embed(_p(ids), _p(emb), _p(r), T, d)
    return r


# ------------------------------------------------------------------ model
# Wiring mutations of OracleModel (tests plant them to show that the
# whole-model fixtures catch each one; never set outside tests):
#   "swap_xz"        the conv takes the z half and the gate the x half
#   "norm_f_v2"      the final norm uses the BitShiftNormV2 table
#   "block_norm_v1"  the SSD block's norm uses the BitShiftNorm table
#   "no_residual"    a block returns out * res_gate without the residual
#   "conv_reset"     the recurrent step forgets the conv ring
#   "no_out_clamp"   the SSD block's out_proj output is not clamped
_WIRING = {"swap_xz", "norm_f_v2", "block_norm_v1", "no_residual", "conv_reset", "no_out_clamp"}
_wiring_mutation: Optional[str] = None


def set_wiring_mutation(m: Optional[str]) -> None:
    global _wiring_mutation
    if m is not None and m not in _WIRING:
        raise ValueError(f"unknown wiring mutation {m!r}")
    _wiring_mutation = m


def _xz_wired(xz: np.ndarray, D: int) -> np.ndarray:
    if _wiring_mutation == "swap_xz":
        return np.ascontiguousarray(np.concatenate([xz[..., D:], xz[..., :D]], axis=-1))
    return xz


def _residual(r: np.ndarray) -> np.ndarray:
    return np.zeros_like(r) if _wiring_mutation == "no_residual" else r


def _conv_in(state: Optional["LayerState"]):
    if state is None or _wiring_mutation == "conv_reset":
        return None
    return state.conv


@dataclass
class LayerState:
    conv: np.ndarray   # int8 [B,3,D]
    h: np.ndarray      # int32 [B,D,N]


class OracleModel:
    """Integer Mamba stack on the CPU oracle (spec rules 4.1-4.12; the SSD
    block of section 7 when dims.block is "ssd")."""

    def __init__(self, params: ModelParams):
        self.p = params
        self.dims = params.dims
        self._wu = {}   # packed matrix -> its int8 unpacking, made on first use

    def _w(self, wp: np.ndarray) -> np.ndarray:
        """The unpacked int8 form of a packed weight matrix of this model (the
        model's parameters do not change during its life)."""
        key = id(wp)
        hit = self._wu.get(key)
        if hit is None or hit[0] is not wp:
            hit = (wp, unpack_ternary(wp, wp.shape[1] * 4))
            self._wu[key] = hit
        return hit[1]

    def _layer(self, lp, r, B, L, state: Optional[LayerState]):
        dm_ = self.dims
        D, N, R = dm_.d_inner, dm_.d_state, dm_.dt_rank
        T = B * L
        if dm_.ssd:
            return self._layer_ssd(lp, r, B, L, state)
        a = bitshift_norm(r, lp.gamma)
        xz = _xz_wired(bitlinear(a, self._w(lp.w_in), OUT_INT8, lp.s_in), D)        # [T, 2D]
        xs, conv_state = conv_squareplus(xz.reshape(B, L, 2 * D), D, lp.conv_w, lp.conv_b, _conv_in(state))
        xp = bitlinear(xs.reshape(T, D), self._w(lp.w_x), OUT_INT8, lp.s_x)          # [T, R+2N]
        dmod = bitlinear(np.ascontiguousarray(xp[:, :R]), self._w(lp.w_dt), OUT_DECAY_MOD, lp.s_dt)
        yo, h = block_scan(xs, dmod.reshape(B, L, D), xp.reshape(B, L, -1), R,
                           xz.reshape(B, L, 2 * D), D, lp.base, lp.k, lp.s_y,
                           None if state is None else state.h)
        r = bitlinear(yo.reshape(T, D), self._w(lp.w_out), OUT_RESIDUAL, residual=_residual(r),
                      res_mult=lp.res_mult, res_shift=lp.res_shift)
        return r, LayerState(conv=conv_state, h=h)

    def _layer_ssd(self, lp, r, B, L, state: Optional[LayerState]):
        """MambaIntegerBlockV2 (spec section 7)."""
        D, T = self.dims.d_inner, B * L
        a = (bitshift_norm if _wiring_mutation == "block_norm_v1" else bitshift_norm_v2)(r, lp.gamma)
        xz = _xz_wired(bitlinear(a, self._w(lp.w_in), OUT_INT8, lp.s_in), D)
        xs, conv_state = conv_squareplus(xz.reshape(B, L, 2 * D), D, lp.conv_w, lp.conv_b, _conv_in(state))
        xp = bitlinear(xs.reshape(T, D), self._w(lp.w_x), OUT_INT8, lp.s_x)
        yo, h = ssd_v2_scan(xs, xp.reshape(B, L, -1), xz.reshape(B, L, 2 * D), D, lp.decay_tab, lp.s_y,
                            self.dims.n_heads, self.dims.d_state, None if state is None else state.h)
        r = bitlinear(yo.reshape(T, D), self._w(lp.w_out), OUT_RESIDUAL, residual=_residual(r),
                      res_mult=lp.res_mult, res_shift=lp.res_shift,
                      res_clamp=0 if _wiring_mutation == "no_out_clamp" else lp.out_clamp)
        return r, LayerState(conv=conv_state, h=h)

    def _run(self, ids, states: Optional[List[LayerState]], last_only: bool):
        ids = np.asarray(ids, dtype=np.int64)
        B, L = ids.shape
        r = embed(ids.reshape(-1), self.p.emb)
        new_states = []
        for i, lp in enumerate(self.p.layers):
            r, st = self._layer(lp, r, B, L, None if states is None else states[i])
            new_states.append(st)
        if last_only:
            r = np.ascontiguousarray(r.reshape(B, L, -1)[:, -1, :])
        a = (bitshift_norm_v2 if _wiring_mutation == "norm_f_v2" else bitshift_norm)(r, self.p.gamma_f)
        logits = bitlinear(a, self._w(self.p.w_head), OUT_INT32)
        return logits, new_states

    def forward(self, ids) -> np.ndarray:
        """All-position int32 logits [B, L, V] (MambaIntegerModel.forward)."""
        ids = np.asarray(ids)
        logits, _ = self._run(ids, None, last_only=False)
        return logits.reshape(ids.shape[0], ids.shape[1], -1)

    def prefill(self, ids, states=None):
        logits, st = self._run(ids, states, last_only=True)
        return logits, st

    def decode_step(self, tokens, states):
        tokens = np.asarray(tokens, dtype=np.int64).reshape(-1, 1)
        logits, st = self._run(tokens, states, last_only=True)
        return logits, st

    def generate(self, ids, n_new: int):
        """Greedy decode (argmax, first maximal index): returns [B, n_new] ids."""
        logits, st = self.prefill(ids)
        out = []
        for _ in range(n_new):
            nxt = np.argmax(logits, axis=-1)
            out.append(nxt)
            logits, st = self.decode_step(nxt, st)
        return np.stack(out, axis=1)
