"""Drop-in for the reference's ``src/mamba_integer_model.py`` on the integer
MI355X path.

Same module names and constructor signatures as the reference
(``MambaIntegerModel(config)``, ``MambaIntegerBlock(config, layer_idx)``,
``BitShiftNorm(dim)``, ``DyadicScanFunction.apply(u, decay_nums,
decay_shifts)``), computing the integer rules of spec mi-spec-2 on the GPU:

- ``MambaIntegerModel.forward(input_ids)`` (``:486-495``) returns float logits
  ``fp32(logit_int) * logit_scale`` (a positive scale, so greedy argmax equals
  the argmax of the exact int32 logits, which ``forward_int`` returns);
- ``generate`` adds the recurrent decode the reference lacks
  (``scripts/inference.py:147-161`` re-runs the whole prefix per token);
- the weights are integer parameters (2-bit ternary, int8, int32 decays),
  built by ``mamba_int.params.init_random_params`` for a synthetic model or
  passed in as ``params``.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn as nn

from mamba_int import checkpoint, ops
from mamba_int.model import IntegerMambaRunner
from mamba_int.params import (DECAY_SHIFT, LayerParams, ModelDims, ModelParams,
                              init_random_params, requant_shift)


class DyadicScanFunction:
    """Integer form of the reference's scan op (``mamba_integer_model.py:260-316``):
    ``h_t = sat32(floor(h_{t-1} * n_t / 2^shift) + u_t)`` over [B, L, C] int32
    tensors, one shift for the whole tensor (as the reference's model uses,
    ``:389``).  Forward only."""

    @staticmethod
    def apply(u: torch.Tensor, decay_nums: torch.Tensor, decay_shifts) -> torch.Tensor:
        if u.dtype != torch.int32 or decay_nums.dtype != torch.int32:
            raise TypeError("the integer scan takes int32 u and decay_nums")
        shift = int(decay_shifts) if not isinstance(decay_shifts, torch.Tensor) \
            else int(decay_shifts.reshape(-1)[0].item())
        return ops.dyadic_scan_elementwise(u.contiguous(), decay_nums.contiguous(), shift)


class BitShiftNorm(nn.Module):
    """Integer BitShiftNorm (spec rule 4.1): int32 Q8 residual -> int8."""

    def __init__(self, dim: int):
        super().__init__()
        self.register_buffer("gamma_q", torch.full((dim,), 256, dtype=torch.int16))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        out = ops.bitshift_norm(x.reshape(-1, shape[-1]).contiguous(), self.gamma_q.to(x.device))
        return out.view(shape)


def _layer_params(dims: ModelDims, rng: np.random.Generator) -> LayerParams:
    one = ModelDims(dims.d_model, 1, 16, dims.d_state, dims.dt_rank, dims.block, dims.n_heads, dims.d_head)
    p = init_random_params(one, int(rng.integers(0, 2**31 - 1)))
    return p.layers[0]


class MambaIntegerBlock(nn.Module):
    """One integer Mamba block (``mamba_integer_model.py:368-447``): int32 Q8
    residual [B, L, d_model] in and out (``residual + out * res_gate`` is the
    saturating int32 residual update of the out_proj epilogue)."""

    def __init__(self, config: dict, layer_idx: int, params: Optional[LayerParams] = None,
                 seed: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.dims = ModelDims.from_config(config)
        self.dims.validate()
        self.params = params if params is not None else _layer_params(
            self.dims, np.random.default_rng(seed * 1000003 + layer_idx))
        self._runner = None

    def _get_runner(self, device) -> IntegerMambaRunner:
        if self._runner is None or self._runner.device != torch.device(device):
            d = self.dims
            mp = ModelParams(dims=ModelDims(d.d_model, 1, 16, d.d_state, d.dt_rank, d.block, d.n_heads, d.d_head),
                             emb=np.zeros((16, d.d_model), np.int8), layers=[self.params],
                             gamma_f=np.full(d.d_model, 256, np.int16),
                             w_head=np.zeros((16, d.d_model // 4), np.uint8))
            self._runner = IntegerMambaRunner(mp, device=str(device))
        return self._runner

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.dtype != torch.int32 or not hidden_states.is_cuda:
            raise TypeError("MambaIntegerBlock takes the int32 Q8 residual stream on the GPU")
        B, L, d = hidden_states.shape
        run = self._get_runner(hidden_states.device)
        ws = run._workspace(B * L)
        ws.r.copy_(hidden_states.reshape(B * L, d))
        st = run.new_state(B)
        run._layer(run.layers[0], ws, B, L, st.conv[0], st.h[0], True, None, None)
        return ws.r.clone().view(B, L, d)


class BitShiftNormV2(BitShiftNorm):
    """Integer BitShiftNormV2 (``ssd_multihead.py:595-632``; spec rule 7.1)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        out = ops.bitshift_norm(x.reshape(-1, shape[-1]).contiguous(), self.gamma_q.to(x.device), v2=True)
        return out.view(shape)


class MambaIntegerBlockV2(MambaIntegerBlock):
    """One integer multi-head SSD block (``ssd_multihead.py:471-592``, selected by
    ``ssm_cfg.use_ssd``): int32 Q8 residual in and out, spec section 7."""

    def __init__(self, config: dict, layer_idx: int, params=None, seed: int = 0):
        cfg = dict(config, ssm_cfg=dict(config.get("ssm_cfg", {}), use_ssd=True))
        super().__init__(cfg, layer_idx, params=params, seed=seed)


class MambaIntegerModel(nn.Module):
    """Integer Mamba language model (``mamba_integer_model.py:466-495``); the
    layers are multi-head SSD blocks when ``ssm_cfg.use_ssd`` is set
    (``:473-476``)."""

    def __init__(self, config: dict, params: Optional[ModelParams] = None, seed: int = 0):
        super().__init__()
        self.config = config
        dims = ModelDims.from_config(config)
        self.params = params if params is not None else init_random_params(dims, seed)
        self.dims = self.params.dims
        self.output_scale = 1.0 / math.sqrt(self.dims.d_model)
        # logits_float = logit_int * 2^-4 (Q4 activations) / sqrt(2K/3) * output_scale
        self.logit_scale = self.output_scale / 16.0 / math.sqrt(2.0 * self.dims.d_model / 3.0)
        self._runner: Optional[IntegerMambaRunner] = None

    @classmethod
    def from_checkpoint(cls, path: str) -> "MambaIntegerModel":
        """The model of a format-1 integer checkpoint (``mamba_int.checkpoint``:
        written by ``save`` or converted from a reference float state dict by
        ``convert_reference_checkpoint``), with its stored logit scale."""
        params, logit_scale = checkpoint.load(path)
        d = params.dims
        config = {"d_model": d.d_model, "n_layer": d.n_layer, "vocab_size": d.vocab_size,
                  "ssm_cfg": {"d_state": d.d_state, "dt_rank": d.dt_rank}}
        model = cls(config, params=params)
        model.logit_scale = logit_scale
        return model

    def runner(self, device="cuda") -> IntegerMambaRunner:
        if self._runner is None or self._runner.device != torch.device(device):
            self._runner = IntegerMambaRunner(self.params, device=str(device))
        return self._runner

    @torch.no_grad()
    def forward_int(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.runner(input_ids.device).forward_logits(input_ids)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        if not input_ids.is_cuda:
            raise ValueError("MambaIntegerModel runs on the GPU; move input_ids to the device")
        return self.forward_int(input_ids).to(torch.float32) * self.logit_scale

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy generation: returns input_ids extended by max_new_tokens ids."""
        new = self.runner(input_ids.device).generate(input_ids, max_new_tokens, use_graph=use_graph)
        return torch.cat([input_ids, new], dim=1)


__all__ = ["MambaIntegerModel", "MambaIntegerBlock", "MambaIntegerBlockV2", "BitShiftNorm", "BitShiftNormV2",
           "DyadicScanFunction",
           "DECAY_SHIFT", "requant_shift"]
