"""The reference's float inference structure on PyTorch-CPU — TEST
INFRASTRUCTURE ONLY (bench.py's cpu_baseline times it; nothing in the
product imports it).

This restates the reference's CPU path as it runs, not the integer rules of
the GPU path: it is the timing baseline "reference-faithful structure", and
its float outputs are compared with nothing.  Per layer it follows
``MambaIntegerBlock.forward`` (``mamba_integer_model.py:396-447``):

- ``BitShiftNorm``: centre, variance, power-of-2 scale from the threshold
  cascade (``:144-184``, ``:200-223``, ``:449-464``);
- ``BitLinear`` in eval mode: ternary weight quantization on every call
  (``rational_bitnet.py:185-188``), per-token absmax activation quantization
  (``:88-111``), ``F.linear`` on the integer-valued fp32 tensors (``:204``)
  and the rescale (``:208``);
- depthwise conv with padding 3 (``:404``), clamp and the Newton-rsqrt
  squareplus (``:80-121``, ``:410-411``);
- x_proj, dt_proj, decay numerators and dt (``:414-427``), the materialized
  ``u`` of shape [B, L, D, N] (``:428-434``);
- the CPU scan loop ``h = d * h + (1 - d) * u`` over time (``:301-316``);
- ``y = h @ C``, the algebraic sigmoid gate, out_proj, residual gate
  (``:440-447``);

and the model is ``MambaIntegerModel.forward`` (``:486-495``): logits at every
position, scaled by 1/sqrt(d_model).  Decoding re-runs the whole prefix for
every new token, as ``scripts/inference.py:147-161`` does.  Weights are random
floats of the reference's shapes (the timing does not depend on their values).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _pow2_scale(var: torch.Tensor) -> torch.Tensor:
    v = var + 1e-9
    s = torch.ones_like(v)
    for thr, val in ((4.0, 0.5), (16.0, 0.25), (64.0, 0.125), (256.0, 0.0625), (1024.0, 0.03125),
                     (4096.0, 0.015625), (16384.0, 0.0078125), (65536.0, 0.00390625)):
        s = torch.where(v >= thr, torch.full_like(s, val), s)
    for thr, val in ((1.0, 1.0), (0.25, 2.0), (0.0625, 4.0), (0.015625, 8.0)):
        s = torch.where(v < thr, torch.full_like(s, val), s)
    return s


def bitshift_norm(x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    x = x - x.mean(dim=-1, keepdim=True)
    xc = x - x.mean(dim=-1, keepdim=True)
    var = xc.pow(2).mean(dim=-1, keepdim=True)
    return xc * _pow2_scale(var) * gamma


def bitlinear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    ws = torch.clamp(w.abs().mean(), min=1e-6)
    wq = torch.clamp(torch.round(w / ws), -1, 1)
    xs = torch.amax(x.abs(), dim=-1, keepdim=True).clamp(min=1e-8)
    xq = torch.round(x * (127.0 / xs)).clamp(-127, 127)
    return F.linear(xq, wq) * (ws * (xs / 127.0))


def squareplus(x: torch.Tensor, iters: int = 3) -> torch.Tensor:
    y = torch.clamp(x * x + 4.0, 1e-6, 1e6)
    r = torch.where(y > 16.0, torch.full_like(y, 0.125), torch.full_like(y, 0.5))
    r = torch.where(y > 64.0, torch.full_like(y, 0.0625), r)
    r = torch.where(y > 256.0, torch.full_like(y, 0.03125), r)
    r = torch.where(y < 4.0, torch.ones_like(y), r)
    r = torch.where(y < 1.0, torch.full_like(y, 2.0), r)
    r = torch.where(y < 0.25, torch.full_like(y, 4.0), r)
    for _ in range(iters):
        r = torch.clamp(r * (1.5 - 0.5 * y * r * r), 1e-6, 1e3)
    return 0.5 * (x + torch.clamp(y * r, 0.0, 1e3))


class RefCpuModel:
    """Float model of the reference's shapes (d_inner = 2 d_model), random init."""

    def __init__(self, d_model: int, n_layer: int, vocab_size: int, d_state: int, dt_rank: int, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        d, D, N, R = d_model, 2 * d_model, d_state, dt_rank
        self.d, self.D, self.N, self.R = d, D, N, R

        def lin(o, i):
            return torch.randn(o, i, generator=g) / math.sqrt(i)
        self.emb = torch.randn(vocab_size, d, generator=g)
        self.layers = []
        for _ in range(n_layer):
            self.layers.append(dict(
                gamma=torch.ones(d), w_in=lin(2 * D, d), conv_w=torch.randn(D, 1, 4, generator=g) * 0.5,
                conv_b=torch.randn(D, generator=g) * 0.1, w_x=lin(R + 2 * N, D), w_dt=lin(D, R),
                w_out=lin(d, D), base=16384.0 + torch.rand(D, N, generator=g) * (32767.0 - 16384.0),
                shifts=torch.full((D, N), 15.0), res_gate=1.0 / math.sqrt(2 * n_layer)))
        self.gamma_f = torch.ones(d)
        self.w_head = lin(vocab_size, d)
        self.out_scale = 1.0 / math.sqrt(d)

    def block(self, P: dict, hs: torch.Tensor) -> torch.Tensor:
        B, L, _ = hs.shape
        D, N, R = self.D, self.N, self.R
        res = hs
        xz = bitlinear(bitshift_norm(hs, P["gamma"]), P["w_in"])
        x, z = xz.chunk(2, dim=-1)
        x = F.conv1d(x.transpose(1, 2), P["conv_w"], P["conv_b"], padding=3, groups=D).transpose(1, 2)[:, :L]
        x = squareplus(torch.clamp(x, -50.0, 50.0))
        dt, Bm, Cm = bitlinear(x, P["w_x"]).split([R, N, N], dim=-1)
        dmod = torch.clamp(bitlinear(dt, P["w_dt"]), -20.0, 20.0)
        nums = torch.clamp(P["base"][None, None] + dmod[..., None], 0, 32000)
        dtv = torch.clamp(squareplus(dmod) * 0.01, 0.001, 0.1)
        u = ((x * dtv)[..., None] * Bm[:, :, None, :]).reshape(B, L, D * N)
        decay = nums.reshape(B, L, D * N) / (2.0 ** P["shifts"].reshape(1, 1, D * N))
        h = torch.zeros(B, D * N)
        hl = []
        for t in range(L):
            h = h * decay[:, t] + (1.0 - decay[:, t]) * u[:, t]
            hl.append(h)
        hseq = torch.stack(hl, dim=1).reshape(B, L, D, N)
        y = torch.matmul(hseq, Cm[..., None]).squeeze(-1)
        y = y * (0.5 + 0.5 * z / (1.0 + z.abs()))
        return res + bitlinear(y, P["w_out"]) * P["res_gate"]

    def forward(self, ids: torch.Tensor, n_layers: int = None) -> torch.Tensor:
        """Logits at every position; n_layers < n_layer runs only the first layers
        (a timing subset)."""
        x = self.emb[ids]
        for P in self.layers[:n_layers]:
            x = self.block(P, x)
        return bitlinear(bitshift_norm(x, self.gamma_f), self.w_head) * self.out_scale
