"""Drop-in for the BitLinear part of the reference's ``src/rational_bitnet.py``
(``:54-231``), backed by libmamba_int.so on the GPU.

Same names, constructor arguments and float-in / float-out contract:

- ``weight_quant_ternary(w)`` (``rational_bitnet.py:63-85``) and
  ``ste_round`` (``:54-60``) are the reference's formulas;
- ``activation_quant_dynamic(x, bits=8)`` (``:88-111``) runs the GPU
  quantizer (IEEE fp32, round half to even), bit-identical to the reference's
  CPU path;
- ``BitLinear.forward`` (``:167-213``) = quantize activations, int8 x ternary
  MFMA product with exact int32 accumulation (what fp32 ``F.linear`` computes
  for these operands), then ``acc * (w_scale * x_scale)`` in fp32, then bias.

The ternary weights and their scale are computed with host (CPU) torch from
``self.weight`` once per weight version (as the reference's cache,
``:181-197``), so ``w_scale`` is the reference CPU value bit for bit; they are
packed 2 bits per weight on the device.  There is no CPU compute path: a
host tensor passed to ``forward`` raises.
"""
from __future__ import annotations

import math
from typing import Tuple

import torch
import torch.nn as nn

from mamba_int import ops


def ste_round(x: torch.Tensor) -> torch.Tensor:
    """Straight-through round (forward value = torch.round(x))."""
    return x + (torch.round(x) - x).detach()


def weight_quant_ternary(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """AbsMean ternary quantization: s = max(mean|W|, 1e-6); Wq = clamp(round(W/s), -1, 1)."""
    scale = torch.max(w.abs().mean(), torch.tensor(1e-6, device=w.device, dtype=w.dtype))
    w_quant = torch.clamp(ste_round(w / scale), min=-1, max=1)
    return w_quant, scale


def activation_quant_dynamic(x: torch.Tensor, bits: int = 8) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token absmax int8 quantization on the GPU; returns (x_quant as fp32, scale/127 [..., 1])."""
    if bits != 8:
        raise ValueError("the integer path quantizes activations to 8 bits")
    if not x.is_cuda:
        raise ValueError("activation_quant_dynamic runs on the GPU; move x to the device")
    shape = x.shape
    q, s = ops.act_quant(x.reshape(-1, shape[-1]).float().contiguous())
    return q.to(torch.float32).view(shape), s.view(*shape[:-1], 1)


def _ceil16(k: int) -> int:
    return (k + 15) // 16 * 16


class BitLinear(nn.Module):
    """Linear layer with {-1, 0, 1} weights and int8 activations (BitNet b1.58)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 activation_bits: int = 8, is_output_layer: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.activation_bits = activation_bits
        self.is_output_layer = is_output_layer
        init_std = 1.0 / math.sqrt(in_features)
        if is_output_layer:
            init_std = init_std / math.sqrt(in_features)
        self.weight = nn.Parameter(torch.randn(out_features, in_features) * init_std)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)
        self._packed = None
        self._w_scale = None
        self._packed_key = None

    # ------------------------------------------------------------ weights
    def _packed_weights(self, device) -> Tuple[torch.Tensor, float]:
        key = (self.weight._version, self.weight.data_ptr(), str(device))
        if self._packed is None or self._packed_key != key:
            w_quant, w_scale = weight_quant_ternary(self.weight.detach().to("cpu", torch.float32))
            k_pad = _ceil16(self.in_features)
            wq = torch.zeros((self.out_features, k_pad), dtype=torch.int8)
            wq[:, : self.in_features] = w_quant.to(torch.int8)
            self._packed = ops.pack_ternary(wq.to(device))
            self._w_scale = float(w_scale)
            self._packed_key = key
        return self._packed, self._w_scale

    @torch.no_grad()
    def get_ternary_weights(self) -> Tuple[torch.Tensor, torch.Tensor]:
        w_quant, w_scale = weight_quant_ternary(self.weight)
        return w_quant.to(torch.int8), w_scale

    # ------------------------------------------------------------ forward
    def _quantized_input(self, x2: torch.Tensor):
        xq, x_scale = ops.act_quant(x2)
        k_pad = _ceil16(self.in_features)
        if k_pad != self.in_features:
            padded = torch.zeros((xq.shape[0], k_pad), dtype=torch.int8, device=xq.device)
            padded[:, : self.in_features] = xq
            xq = padded
        return xq, x_scale

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise ValueError("BitLinear runs on the GPU; move the input to the device")
        if self.activation_bits != 8:
            raise ValueError("the integer path quantizes activations to 8 bits")
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).to(torch.float32).contiguous()
        packed, w_scale = self._packed_weights(x.device)
        xq, x_scale = self._quantized_input(x2)
        y = ops.bitlinear(xq, packed, ops.OUT_FLOAT, self.out_features, x_scale=x_scale, w_scale=w_scale)
        if self.bias is not None:
            y = y + self.bias.to(y.device)
        return y.view(*shape[:-1], self.out_features)

    @torch.no_grad()
    def forward_int(self, a: torch.Tensor, kind: int = ops.OUT_INT32, shift: int = 0) -> torch.Tensor:
        """Integer face: a int8 [M, K] (K = in_features padded to 16) -> acc / requantized int8."""
        packed, _ = self._packed_weights(a.device)
        return ops.bitlinear(a.contiguous(), packed, kind, self.out_features, shift=shift)
