"""The whole decode step behind the C ABI (``mi_decode_step``): ctypes mirrors
of ``mi_layer_params`` / ``mi_model_params`` and a small decoder object that
owns the workspace and the state pointer arrays.

This is the entry a non-Python host (a C++ engine in place of
``src/cpp_engine/mamba_infer.cpp``) would call; from Python it runs one greedy
step per call, enqueued on the current stream (capturable in a HIP graph).
"""
from __future__ import annotations

import ctypes
from typing import List

import torch

from . import _lib

_P = ctypes.c_void_p
_I = ctypes.c_int


class LayerParams(ctypes.Structure):
    """Field-for-field mirror of ``mi_layer_params`` (include/mamba_int.h)."""
    _fields_ = [("gamma", _P), ("w_in", _P), ("s_in", _I), ("conv_w", _P), ("conv_b", _P),
                ("w_x", _P), ("s_x", _I), ("w_dt", _P), ("s_dt", _I), ("base", _P),
                ("decay_shift", _I), ("s_y", _I), ("w_out", _P), ("res_mult", ctypes.c_int32),
                ("res_shift", _I), ("decay_tab", _P), ("out_clamp", ctypes.c_int32)]


class ModelParams(ctypes.Structure):
    """Mirror of ``mi_model_params``; ``layers`` points at a host array."""
    _fields_ = [("d_model", _I), ("n_layer", _I), ("vocab_size", _I), ("d_state", _I), ("dt_rank", _I),
                ("emb", _P), ("layers", ctypes.POINTER(LayerParams)), ("gamma_f", _P), ("w_head", _P),
                ("block", _I), ("n_heads", _I), ("d_head", _I)]


MI_BLOCK_DYADIC, MI_BLOCK_SSD = 0, 1


class CheckpointInfo(ctypes.Structure):
    """Mirror of ``mi_checkpoint_info``."""
    _fields_ = [("format_version", _I), ("spec", ctypes.c_char * 16), ("d_model", _I), ("n_layer", _I),
                ("vocab_size", _I), ("d_state", _I), ("dt_rank", _I), ("logit_scale", ctypes.c_float),
                ("device_bytes", ctypes.c_size_t), ("block", _I), ("n_heads", _I), ("d_head", _I)]


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


class NativeCheckpoint:
    """An integer checkpoint read and validated by the native loader
    (``mi_checkpoint_open``) and, with a device, uploaded into one device
    buffer (``mi_checkpoint_upload``) that ``params`` points into: the C++
    engine's ``load_model`` (``src/cpp_engine/mamba_infer.cpp:46-118``) with
    status codes instead of exit() and no allocation inside the library."""

    def __init__(self, path: str, device=None):
        ck = _P()
        _lib.call("mi_checkpoint_open", str(path).encode(), ctypes.byref(ck))
        try:
            self.info = CheckpointInfo()
            _lib.call("mi_checkpoint_get_info", ck, ctypes.byref(self.info))
            self.params = None
            if device is not None:
                n = self.info.n_layer
                self.buffer = torch.empty(self.info.device_bytes, dtype=torch.uint8, device=device)
                self._layers = (LayerParams * n)()
                self.params = ModelParams()
                _lib.call("mi_checkpoint_upload", ck, _P(_ptr(self.buffer)), ctypes.c_size_t(self.info.device_bytes),
                          ctypes.byref(self.params), self._layers, n,
                          _P(torch.cuda.current_stream(self.buffer.device).cuda_stream))
        finally:
            _lib.load().mi_checkpoint_close(ck)

    def decoder(self, m: int) -> "NativeDecoder":
        if self.params is None:
            raise ValueError("the checkpoint was opened without a device")
        return NativeDecoder.from_params(self.params, self.buffer.device, m, owner=self)


class NativeDecoder:
    """Greedy decode through ``mi_decode_step`` at batch m (1 <= m <= 64), for
    the device parameters of an ``IntegerMambaRunner`` or of a
    ``NativeCheckpoint`` (``from_params``)."""

    def __init__(self, runner, m: int):
        dims = runner.dims
        layers = (LayerParams * dims.n_layer)()
        opt = lambda t: None if t is None else _ptr(t)  # noqa: E731
        for i, ly in enumerate(runner.layers):
            layers[i] = LayerParams(_ptr(ly.gamma), _ptr(ly.w_in), ly.s_in, _ptr(ly.conv_w), _ptr(ly.conv_b),
                                    _ptr(ly.w_x), ly.s_x, opt(ly.w_dt), ly.s_dt, opt(ly.base), ly.k, ly.s_y,
                                    _ptr(ly.w_out), ly.res_mult, ly.res_shift, opt(ly.decay_tab), ly.out_clamp)
        params = ModelParams(dims.d_model, dims.n_layer, dims.vocab_size, dims.d_state, dims.dt_rank,
                             _ptr(runner.emb), layers, _ptr(runner.gamma_f), _ptr(runner.w_head),
                             MI_BLOCK_SSD if dims.ssd else MI_BLOCK_DYADIC, dims.n_heads, dims.d_head)
        self._setup(params, runner.device, m, owner=(runner, layers))

    @classmethod
    def from_params(cls, params: ModelParams, device, m: int, owner=None) -> "NativeDecoder":
        self = cls.__new__(cls)
        self._setup(params, device, m, owner)
        return self

    def _setup(self, params: ModelParams, device, m: int, owner) -> None:
        self.owner, self.m, self.params = owner, m, params  # owner keeps the device tensors alive
        self._pp = ctypes.cast(ctypes.pointer(self.params), _P)
        nbytes = ctypes.c_size_t(0)
        _lib.call("mi_decode_workspace_size", self._pp, m, ctypes.cast(ctypes.pointer(nbytes), _P))
        self.ws_bytes = nbytes.value
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)

    def step(self, ids: torch.Tensor, state, next_ids: torch.Tensor, logits=None) -> torch.Tensor:
        """One step: ids [m] int64 -> next_ids [m] int64 (and int32 logits [m, V] when given);
        ``state`` (a DecodeState of batch m) is updated in place."""
        n = self.params.n_layer
        conv = (ctypes.c_void_p * n)(*[_ptr(c) for c in state.conv])
        h = (ctypes.c_void_p * n)(*[_ptr(t) for t in state.h])
        ld = 0 if logits is None else logits.stride(0)
        _lib.call("mi_decode_step", self._pp, self.m, _P(_ptr(ids)), _P(_ptr(next_ids)),
                  _P(_ptr(logits)) if logits is not None else None, ld, ctypes.cast(conv, _P), ctypes.cast(h, _P),
                  _P(_ptr(self.workspace)), ctypes.c_size_t(self.ws_bytes),
                  _P(torch.cuda.current_stream().cuda_stream))
        return next_ids

    def generate(self, first: torch.Tensor, state, n: int) -> torch.Tensor:
        """n greedy steps from pick `first` [m]: returns [m, n] (column 0 = first)."""
        out = torch.empty((self.m, n), dtype=torch.int64, device=first.device)
        cur = first.clone()
        nxt = torch.empty_like(cur)
        out[:, 0] = cur
        for i in range(1, n):
            self.step(cur, state, nxt)
            out[:, i] = nxt
            cur, nxt = nxt, cur
        return out
