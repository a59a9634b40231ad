"""Integer parameters of the integer Mamba model (spec mi-spec-2).

The reference keeps float parameters and quantizes at run time
(``rational_bitnet.py:185-188``); the integer path stores what that
quantization produces: 2-bit packed ternary matrices, int8 embedding and conv
taps, int32 decay numerators, and the per-layer power-of-2 shifts.

Config keys follow the reference schema (``configs/config_mamba_integer_l4.json``;
``MambaIntegerBlock.__init__``, ``mamba_integer_model.py:369-394``):
``d_model``, ``n_layer``, ``vocab_size``, ``ssm_cfg.{d_state, dt_rank}``;
``d_inner = 2 * d_model`` as ``mamba_integer_model.py:373``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List

import numpy as np

DECAY_SHIFT = 15          # decay_shifts buffer value (mamba_integer_model.py:389)
DECAY_MAX = 32000         # clamp of decay_nums (mamba_integer_model.py:424)
R_LIM = (1 << 23) - 1     # residual saturation
EMB_SHIFT = 4             # r0 = emb << 4 (Q4 -> Q8)


@dataclass
class ModelDims:
    """Model sizes.  block "dyadic": MambaIntegerBlock (d_inner = 2 d_model,
    ``mamba_integer_model.py:373``); block "ssd": MambaIntegerBlockV2 with
    n_heads heads of d_head channels (d_inner = n_heads * d_head,
    ``ssd_multihead.py:489-493``; dt_rank unused)."""
    d_model: int
    n_layer: int
    vocab_size: int
    d_state: int
    dt_rank: int
    block: str = "dyadic"
    n_heads: int = 0
    d_head: int = 0

    @property
    def ssd(self) -> bool:
        return self.block == "ssd"

    @property
    def d_inner(self) -> int:
        return self.n_heads * self.d_head if self.ssd else 2 * self.d_model

    @property
    def xp_width(self) -> int:
        """x_proj output width: dt_rank + 2N, or for the SSD block the planar
        [B (H*N) | C (H*N) | dt (H)] rounded up to a multiple of 16."""
        if self.ssd:
            return -(-(2 * self.n_heads * self.d_state + self.n_heads) // 16) * 16
        return self.dt_rank + 2 * self.d_state

    @staticmethod
    def from_config(config: dict) -> "ModelDims":
        ssm = config.get("ssm_cfg", {})
        d_model = int(config["d_model"])
        if ssm.get("use_ssd", False):
            # MambaIntegerBlockV2 defaults (ssd_multihead.py:489-491)
            return ModelDims(d_model=d_model, n_layer=int(config["n_layer"]),
                             vocab_size=int(config["vocab_size"]), d_state=int(ssm.get("d_state", 64)),
                             dt_rank=0, block="ssd", n_heads=int(ssm.get("n_heads", 24)),
                             d_head=int(ssm.get("d_head", 64)))
        dt_rank = ssm.get("dt_rank")
        if dt_rank is None:
            dt_rank = -(-d_model // 16)
        return ModelDims(d_model=d_model, n_layer=int(config["n_layer"]),
                         vocab_size=int(config["vocab_size"]),
                         d_state=int(ssm.get("d_state", 16)), dt_rank=int(dt_rank))

    def validate(self) -> None:
        checks = [("d_model", self.d_model), ("d_inner", self.d_inner)]
        if not self.ssd:
            checks.append(("dt_rank", self.dt_rank))
        for name, v in checks:
            if v % 16 != 0:
                raise ValueError(f"{name}={v} must be a multiple of 16 (2-bit packing unit)")
        if self.block not in ("dyadic", "ssd"):
            raise ValueError(f"block={self.block!r} (dyadic or ssd)")
        if self.ssd:
            if self.n_heads < 1 or self.d_head < 16 or self.d_head % 16:
                raise ValueError(f"n_heads={self.n_heads}, d_head={self.d_head}: d_head a multiple of 16")
            if self.d_state not in (16, 32, 64):
                raise ValueError(f"d_state={self.d_state}: the SSD block takes 16, 32 or 64")
        elif not (1 <= self.d_state <= 64):
            raise ValueError(f"d_state={self.d_state} outside [1, 64]")


def requant_shift(k: int) -> int:
    """Initial power-of-2 requant shift for fan-in k: floor(log2(2k/3)/2)."""
    return max(0, int(math.floor(math.log2(2.0 * k / 3.0) / 2.0)))


def _bitpos() -> np.ndarray:
    q = np.arange(16)
    return 8 * (q & 3) + 2 * (q >> 2)


def pack_ternary(w: np.ndarray) -> np.ndarray:
    """int8 {-1,0,1} [N,K] -> uint8 [N,K/4]: K/16 little-endian words per row,
    weight 16w+4j+i at bits [8i+2j, 8i+2j+1] of word w; codes 0->00, +1->01,
    -1->11."""
    w = np.asarray(w)
    n, k = w.shape
    if k % 16:
        raise ValueError("K must be a multiple of 16")
    if np.any((w < -1) | (w > 1)):
        raise ValueError("ternary weights must lie in {-1, 0, 1}")
    code = (w.astype(np.int8).view(np.uint8) & 3).astype(np.uint32).reshape(n, k // 16, 16)
    words = np.bitwise_or.reduce(code << _bitpos().astype(np.uint32), axis=-1).astype("<u4")
    return words.view(np.uint8).reshape(n, k // 4)


def unpack_ternary(p: np.ndarray, k: int) -> np.ndarray:
    p = np.ascontiguousarray(p, dtype=np.uint8)
    n = p.shape[0]
    words = p.reshape(n, k // 16, 4).view("<u4")[..., 0].astype(np.int64)
    codes = (words[..., None] >> _bitpos()) & 3
    vals = np.where(codes >= 2, codes - 4, codes).astype(np.int8)
    return vals.reshape(n, k)


@dataclass
class LayerParams:
    gamma: np.ndarray        # int16 [d] Q8
    w_in: np.ndarray         # uint8 [2D, d/4]
    s_in: int
    conv_w: np.ndarray       # int8 [D, 4] Q6
    conv_b: np.ndarray       # int32 [D] Q10
    w_x: np.ndarray          # uint8 [R+2N, D/4]
    s_x: int
    w_dt: np.ndarray         # uint8 [D, R/4]
    s_dt: int
    base: np.ndarray         # int32 [D, N]
    k: int
    s_y: int
    w_out: np.ndarray        # uint8 [d, D/4]
    res_mult: int
    res_shift: int
    out_clamp: int = 0       # MambaIntegerBlock has no out_proj clamp


@dataclass
class SSDLayerParams:
    """One MambaIntegerBlockV2 layer (spec section 7)."""
    gamma: np.ndarray        # int16 [d] Q8 (V2 norm table)
    w_in: np.ndarray         # uint8 [2D, d/4]
    s_in: int
    conv_w: np.ndarray       # int8 [D, 4] Q6
    conv_b: np.ndarray       # int32 [D] Q10
    w_x: np.ndarray          # uint8 [xp_width, D/4], planar rows [B | C | dt | 0]
    s_x: int
    decay_tab: np.ndarray    # int32 [H, 255]: decay numerator per head and dt in [-127, 127]
    s_y: int
    w_out: np.ndarray        # uint8 [d, D/4]
    res_mult: int
    res_shift: int
    out_clamp: int           # out_proj accumulator bound (spec rule 7.9), >= 1
    k: int = DECAY_SHIFT


def out_clamp_for(w_scale: float) -> int:
    """The SSD block's out_proj clamp (spec rule 7.9) for an out_proj weight scale:
    out = acc * w_scale / 16 (Q4 input) lies in [-100, 100] (``ssd_multihead.py:589-590``)
    exactly when |acc| <= floor(1600 / w_scale)."""
    if not w_scale > 0:
        raise ValueError("the out_proj weight scale must be positive")
    return int(min(2**31 - 1, max(1, math.floor(1600.0 / w_scale))))


def synthetic_out_clamp(n_layer: int, res_mult: int, res_shift: int) -> int:
    """out_clamp_for the weight scale a synthetic layer's (res_mult, res_shift) stands
    for under the reference's initial res_gate 1/sqrt(2 n_layer) (``ssd_multihead.py:518``):
    res_mult / 2^res_shift = 16 * w_scale * res_gate."""
    res_gate = 1.0 / math.sqrt(2.0 * n_layer)
    return out_clamp_for(res_mult / 2.0**res_shift / (16.0 * res_gate))


def ssd_decay_table(a_log) -> np.ndarray:
    """Per-head decay numerators of the SSD block (spec rule 7.5), float64:
    A = clamp(clamp(A_log, -2.3, -0.01) * clamp(softplus(clamp(dt, +-10)),
    0.01, 10), -20, -0.001) for dt = q/16, q in [-127, 127]
    (``ssd_multihead.py:555-570``); entry = round_half_even(exp(A) * 2^15)."""
    a = np.clip(np.asarray(a_log, dtype=np.float64).reshape(-1, 1), -2.3, -0.01)
    dt = np.clip(np.arange(-127, 128, dtype=np.float64) / 16.0, -10.0, 10.0)
    sp = np.clip(np.logaddexp(0.0, dt), 0.01, 10.0)
    A = np.clip(a * sp[None, :], -20.0, -0.001)
    return np.round(np.exp(A) * 32768.0).astype(np.int32)


@dataclass
class ModelParams:
    dims: ModelDims
    emb: np.ndarray          # int8 [V, d] Q4
    layers: List[LayerParams] = field(default_factory=list)
    gamma_f: np.ndarray = None   # int16 [d]
    w_head: np.ndarray = None    # uint8 [V, d/4]


def _ternary(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    return pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))


def init_random_params(dims: ModelDims, seed: int) -> ModelParams:
    """Random integer model: ternary weights i.i.d. in {-1,0,1} with p=1/3,
    decays uniform [16384, 32000] with shift 15 (a synthetic checkpoint); for
    the SSD block, per-head A_log uniform in [-2.3, -0.01] and the padding
    rows of x_proj zero."""
    dims.validate()
    rng = np.random.default_rng(seed)
    d, D, N, R, V = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank, dims.vocab_size
    emb = rng.integers(-64, 65, size=(V, d), dtype=np.int8)
    layers = []
    if dims.ssd:
        H, W = dims.n_heads, dims.xp_width
        for _ in range(dims.n_layer):
            wx = rng.integers(-1, 2, size=(W, D), dtype=np.int8)
            wx[2 * H * N + H:] = 0
            layers.append(SSDLayerParams(
                gamma=np.full(d, 256, dtype=np.int16),
                w_in=_ternary(rng, 2 * D, d), s_in=requant_shift(d),
                conv_w=rng.integers(-32, 33, size=(D, 4), dtype=np.int8),
                conv_b=rng.integers(-512, 513, size=D, dtype=np.int32),
                w_x=pack_ternary(wx), s_x=requant_shift(D),
                decay_tab=ssd_decay_table(rng.uniform(-2.3, -0.01, size=H)), s_y=14,
                w_out=_ternary(rng, d, D), res_mult=4719, res_shift=16,
                out_clamp=synthetic_out_clamp(dims.n_layer, 4719, 16)))
        return ModelParams(dims=dims, emb=emb, layers=layers, gamma_f=np.full(d, 256, dtype=np.int16),
                           w_head=_ternary(rng, V, d))
    for _ in range(dims.n_layer):
        layers.append(LayerParams(
            gamma=np.full(d, 256, dtype=np.int16),
            w_in=_ternary(rng, 2 * D, d), s_in=requant_shift(d),
            conv_w=rng.integers(-32, 33, size=(D, 4), dtype=np.int8),
            conv_b=rng.integers(-512, 513, size=D, dtype=np.int32),
            w_x=_ternary(rng, R + 2 * N, D), s_x=requant_shift(D),
            w_dt=_ternary(rng, D, R), s_dt=requant_shift(R) + 3,
            base=rng.integers(16384, 32001, size=(D, N), dtype=np.int32),
            k=DECAY_SHIFT, s_y=14,
            w_out=_ternary(rng, d, D), res_mult=4719, res_shift=16,
        ))
    return ModelParams(dims=dims, emb=emb, layers=layers,
                       gamma_f=np.full(d, 256, dtype=np.int16),
                       w_head=_ternary(rng, V, d))
