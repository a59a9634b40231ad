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
  built by ``mamba_int.params.init_random_params`` for a synthetic model (on
  first use), passed in as ``params``, read from an integer checkpoint
  (``from_checkpoint``), or converted from the reference's float state dict
  by ``load_state_dict`` as ``scripts/inference.py:103-121`` calls it;
- ``MambaIntegerBlock.forward`` and ``BitShiftNorm.forward`` take the
  reference's float tensors (quantized to the Q8 residual on entry, returned
  as floats) or the int32 Q8 residual itself (``forward_int``).
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn as nn
from torch.nn.modules.module import _IncompatibleKeys

from mamba_int import checkpoint, ops
from mamba_int.model import IntegerMambaRunner
from mamba_int.params import (DECAY_SHIFT, LayerParams, ModelDims, ModelParams,
                              init_random_params, requant_shift, synthetic_out_clamp)


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


RESIDUAL_LIMIT = (1 << 23) - 1     # the Q8 residual saturates at +-(2^23 - 1)


def to_q8(x: torch.Tensor) -> torch.Tensor:
    """Float hidden states -> the int32 Q8 residual: round_half_even(x * 256)
    (exact scaling in fp32), saturated to +-(2^23 - 1)."""
    q = torch.round(x.to(torch.float32) * 256.0)
    return q.clamp_(-RESIDUAL_LIMIT, RESIDUAL_LIMIT).to(torch.int32)


class BitShiftNorm(nn.Module):
    """Integer BitShiftNorm (spec rule 4.1; ``mamba_integer_model.py:449-464``).
    ``forward_int``: int32 Q8 residual -> int8 Q4.  ``forward`` on a float tensor
    quantizes it to Q8 and returns the int8 result as floats (value / 16);
    on int32 it is ``forward_int``.  The gain is gamma * step_size in Q8."""

    _V2 = False

    def __init__(self, dim: int):
        super().__init__()
        self.dim = dim
        self.register_buffer("gamma_q", torch.full((dim,), 256, dtype=torch.int16))

    def forward_int(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        out = ops.bitshift_norm(x.reshape(-1, shape[-1]).contiguous(), self.gamma_q.to(x.device), v2=self._V2)
        return out.view(shape)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype == torch.int32:
            return self.forward_int(x)
        if not x.is_floating_point():
            raise TypeError("BitShiftNorm takes float hidden states or the int32 Q8 residual")
        return self.forward_int(to_q8(x)).to(torch.float32) * (1.0 / 16.0)

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """The reference's ``gamma`` [dim] and ``step_size`` [1] (or this module's own
        ``gamma_q``): gamma_q = clamp(round_half_even(gamma * step_size * 256), +-32767)."""
        sd = dict(state_dict)
        if "gamma_q" in sd:
            q = torch.as_tensor(sd.pop("gamma_q"))
            if q.shape != (self.dim,):
                raise ValueError(f"gamma_q: shape {tuple(q.shape)}, want ({self.dim},)")
            self.gamma_q = q.to(torch.int16).to(self.gamma_q.device)
        else:
            if "gamma" not in sd or "step_size" not in sd:
                raise KeyError("BitShiftNorm state dict needs gamma and step_size")
            g = torch.as_tensor(sd.pop("gamma"), dtype=torch.float32).cpu()
            st = torch.as_tensor(sd.pop("step_size"), dtype=torch.float32).cpu().reshape(-1)
            if g.shape != (self.dim,) or st.numel() != 1:
                raise ValueError(f"gamma {tuple(g.shape)} / step_size {tuple(st.shape)} do not fit dim {self.dim}")
            q = torch.round(g * st[0] * 256.0).clamp(-32767, 32767).to(torch.int16)
            self.gamma_q = q.to(self.gamma_q.device)
        unexpected = sorted(sd)
        if strict and unexpected:
            raise RuntimeError(f"Unexpected key(s) in state_dict: {unexpected}")
        return _IncompatibleKeys([], unexpected)


def _layer_params(dims: ModelDims, rng: np.random.Generator) -> LayerParams:
    one = ModelDims(dims.d_model, 1, 16, dims.d_state, dims.dt_rank, dims.block, dims.n_heads, dims.d_head)
    ly = init_random_params(one, int(rng.integers(0, 2**31 - 1))).layers[0]
    if dims.ssd:     # the synthetic out clamp of a layer in an n_layer-deep model
        ly.out_clamp = synthetic_out_clamp(dims.n_layer, ly.res_mult, ly.res_shift)
    return ly


class MambaIntegerBlock(nn.Module):
    """One integer Mamba block (``mamba_integer_model.py:368-447``).
    ``forward(hidden_states)`` takes the reference's float [B, L, d_model]
    hidden states, quantizes them to the Q8 residual (``to_q8``), runs the
    integer block and returns the new residual as floats (value / 256);
    ``forward_int`` (and ``forward`` on int32) runs on the int32 Q8 residual
    itself (``residual + out * res_gate`` is the saturating int32 residual
    update of the out_proj epilogue)."""

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

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """The reference block's float state dict (``in_proj.weight``, ``conv1d.*``,
        ``norm.gamma``, ...; no ``layers.{i}.`` prefix) converted to integers by
        ``mamba_int.checkpoint.convert_block_state_dict``.  A tensor the block
        needs that is missing, a wrong shape or a value the integer block cannot
        represent raises ``CheckpointError`` whatever ``strict`` is; keys it does
        not use raise under ``strict`` and are returned as unexpected otherwise."""
        layer, unused = checkpoint.convert_block_state_dict(state_dict, self.config)
        if strict and unused:
            raise RuntimeError(f"Unexpected key(s) in state_dict: {unused[:5]}")
        self.params = layer
        self._runner = None
        return _IncompatibleKeys([], unused)

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.dtype == torch.int32:
            return self.forward_int(hidden_states)
        if not hidden_states.is_floating_point():
            raise TypeError("MambaIntegerBlock takes float hidden states or the int32 Q8 residual")
        return self.forward_int(to_q8(hidden_states)).to(torch.float32) * (1.0 / 256.0)

    @torch.no_grad()
    def forward_int(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.dtype != torch.int32 or not hidden_states.is_cuda:
            raise TypeError("forward_int takes the int32 Q8 residual stream on the GPU")
        B, L, d = hidden_states.shape
        run = self._get_runner(hidden_states.device)
        ws = run._workspace(B * L)
        ws.r.copy_(hidden_states.reshape(B * L, d))
        st = run.new_state(B)
        run._layer(run.layers[0], ws, B, L, st.conv[0], st.h[0], True, None, None)
        return ws.r.clone().view(B, L, d)


class BitShiftNormV2(BitShiftNorm):
    """Integer BitShiftNormV2 (``ssd_multihead.py:595-632``; spec rule 7.1)."""

    _V2 = True


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
        self._seed = seed
        self._params = params
        self.dims = params.dims if params is not None else ModelDims.from_config(config)
        self.dims.validate()
        self.output_scale = 1.0 / math.sqrt(self.dims.d_model)
        # logits_float = logit_int * 2^-4 (Q4 activations) / sqrt(2K/3) * output_scale
        self.logit_scale = self.output_scale / 16.0 / math.sqrt(2.0 * self.dims.d_model / 3.0)
        self._runner: Optional[IntegerMambaRunner] = None

    @property
    def params(self) -> ModelParams:
        """The integer parameters; a synthetic random model (seeded) is built on
        first use when none were given or loaded."""
        if self._params is None:
            self._params = init_random_params(self.dims, self._seed)
        return self._params

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """Loads the reference's float ``MambaIntegerModel`` state dict (keys of
        ``mamba_integer_model.py:368-394,449-484``; ``ssd_multihead.py:481-522``
        for ``use_ssd``), as ``scripts/inference.py:103-121`` does after
        ``MambaIntegerModel(config)``: ``_orig_mod.`` / ``module.`` prefixes are
        stripped, the tensors are converted to the integer parameters and the
        logit scale by ``mamba_int.checkpoint.convert_state_dict``, and they
        replace the model's (the GPU runner is rebuilt on next use).

        A tensor the model needs that is missing, a shape that disagrees with
        the config or a value the integer model cannot represent raises
        ``CheckpointError`` whatever ``strict`` is: the model never keeps
        random weights silently.  Keys the integer model does not use raise
        ``RuntimeError`` under ``strict`` and are returned as
        ``unexpected_keys`` otherwise (``missing_keys`` is always empty)."""
        params, logit_scale, unused = checkpoint.convert_state_dict_keys(state_dict, self.config)
        if strict and unused:
            raise RuntimeError(f"Unexpected key(s) in state_dict: {unused[:5]}")
        self._params = params
        self.dims = params.dims
        self.logit_scale = logit_scale
        self._runner = None
        return _IncompatibleKeys([], unused)

    @classmethod
    def from_checkpoint(cls, path: str) -> "MambaIntegerModel":
        """The model of an integer checkpoint (``mamba_int.checkpoint``: written by
        ``save`` or converted from a reference float state dict by
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
