"""Device runner of the integer Mamba stack (spec rules 4.1-4.12).

Orchestrates the per-layer kernels in the block order of
``MambaIntegerBlock.forward`` (``mamba_integer_model.py:396-447``) and the
model order of ``MambaIntegerModel.forward`` (``:486-495``).  Adds what the
reference lacks: a recurrent decode step with per-layer conv and scan state
(the reference recomputes the whole prefix per token,
``scripts/inference.py:147-161``), and a HIP-graph-captured greedy decode loop.

Activations live in preallocated int8/int32 workspaces sized for one
(batch, length); the int32 residual is updated in place by the out_proj
epilogue.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import ops
from .params import LayerParams, ModelParams


@dataclass
class DeviceLayer:
    """Device parameters of one layer: the dyadic-scan block uses w_dt, s_dt
    and base, the SSD block its per-head decay table."""
    gamma: torch.Tensor
    w_in: torch.Tensor
    s_in: int
    conv_w: torch.Tensor
    conv_b: torch.Tensor
    w_x: torch.Tensor
    s_x: int
    s_y: int
    w_out: torch.Tensor
    res_mult: int
    res_shift: int
    out_clamp: int = 0
    k: int = 15
    w_dt: Optional[torch.Tensor] = None
    s_dt: int = 0
    base: Optional[torch.Tensor] = None
    decay_tab: Optional[torch.Tensor] = None


@dataclass
class DecodeState:
    """Recurrent state of every layer: conv ring [B,3,D] int8, scan state [B,D,N] int32."""
    conv: List[torch.Tensor]
    h: List[torch.Tensor]

    def clone(self) -> "DecodeState":
        return DecodeState([c.clone() for c in self.conv], [h.clone() for h in self.h])


def _dev(a, device) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a.to(device)
    return torch.from_numpy(a.copy()).to(device)


def random_device_params(dims, seed: int, device: str = "cuda") -> ModelParams:
    """A synthetic integer model generated on the device (same distributions as
    params.init_random_params, different draws): ternary weights i.i.d. in
    {-1,0,1} packed by mi_pack_ternary, decays uniform [16384, 32000].  For
    benchmarks of large configurations, where drawing 10^9 weights on the host
    would take minutes."""
    from .params import DECAY_SHIFT, requant_shift
    dims.validate()
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    d, D, N, R, V = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank, dims.vocab_size

    def ri(lo, hi, shape, dtype):
        return torch.randint(lo, hi + 1, shape, generator=g, device=dev, dtype=torch.int64).to(dtype)

    def tern(n, k):
        return ops.pack_ternary(ri(-1, 1, (n, k), torch.int8))

    layers = []
    for _ in range(dims.n_layer):
        layers.append(LayerParams(
            gamma=torch.full((d,), 256, dtype=torch.int16, device=dev), w_in=tern(2 * D, d), s_in=requant_shift(d),
            conv_w=ri(-32, 32, (D, 4), torch.int8), conv_b=ri(-512, 512, (D,), torch.int32),
            w_x=tern(R + 2 * N, D), s_x=requant_shift(D), w_dt=tern(D, R), s_dt=requant_shift(R) + 3,
            base=ri(16384, 32000, (D, N), torch.int32), k=DECAY_SHIFT, s_y=14,
            w_out=tern(d, D), res_mult=4719, res_shift=16))
    return ModelParams(dims=dims, emb=ri(-64, 64, (V, d), torch.int8), layers=layers,
                       gamma_f=torch.full((d,), 256, dtype=torch.int16, device=dev), w_head=tern(V, d))


class _Workspace:
    def __init__(self, dims, T: int, device):
        D, d = dims.d_inner, dims.d_model
        self.T = T
        self.r = torch.empty((T, d), dtype=torch.int32, device=device)
        self.a = torch.empty((T, d), dtype=torch.int8, device=device)
        self.xz = torch.empty((T, 2 * D), dtype=torch.int8, device=device)
        self.xs = torch.empty((T, D), dtype=torch.int8, device=device)
        self.xp = torch.empty((T, dims.xp_width), dtype=torch.int8, device=device)
        self.dm = torch.empty((T, D), dtype=torch.int8, device=device)
        self.yo = torch.empty((T, D), dtype=torch.int8, device=device)
        # row statistics (sum r, sum r^2) of the residual entering layer i (i = n_layer: the head)
        self.stats = torch.empty((dims.n_layer + 1, T, 2), dtype=torch.int64, device=device)
        # decode (T <= 16): per-16-feature row-statistics partials of the out_proj,
        # summed by the next norm (one buffer: each norm reads it before its
        # layer's out_proj rewrites it)
        self.parts = (torch.empty((T, d // 16, 2), dtype=torch.int64, device=device)
                      if T <= 64 and d % 16 == 0 else None)
        # x_proj partials of the decode chain (one row per 16 channels of d_inner)
        nx = dims.dt_rank + 2 * dims.d_state
        self.xpart = (torch.empty((T, D // 16, nx), dtype=torch.int32, device=device)
                      if T <= 64 and (D // 16) * nx <= 8192 else None)
        # the batched decode step's x_proj sums over the four channel quarters
        self.xq = (torch.empty((T, 4, nx), dtype=torch.int32, device=device)
                   if T <= 1024 and D % 1024 == 0 and D <= 8192 and nx <= 256 else None)


class IntegerMambaRunner:
    def __init__(self, params: ModelParams, device: str = "cuda"):
        self.dims = params.dims
        self.dims.validate()
        if self.dims.xp_width % 16 or self.dims.dt_rank % 16:
            raise ValueError("dt_rank and dt_rank + 2*d_state must be multiples of 16")
        self.device = torch.device(device)
        dv = self.device
        self.emb = _dev(params.emb, dv)
        self.layers: List[DeviceLayer] = []
        for lp in params.layers:
            common = dict(gamma=_dev(lp.gamma, dv), w_in=_dev(lp.w_in, dv), s_in=lp.s_in,
                          conv_w=_dev(lp.conv_w, dv), conv_b=_dev(lp.conv_b, dv), w_x=_dev(lp.w_x, dv),
                          s_x=lp.s_x, k=lp.k, s_y=lp.s_y, w_out=_dev(lp.w_out, dv), res_mult=lp.res_mult,
                          res_shift=lp.res_shift, out_clamp=lp.out_clamp)
            if self.dims.ssd:
                self.layers.append(DeviceLayer(**common, decay_tab=_dev(lp.decay_tab, dv)))
            else:
                self.layers.append(DeviceLayer(**common, w_dt=_dev(lp.w_dt, dv), s_dt=lp.s_dt,
                                               base=_dev(lp.base, dv)))
        self.gamma_f = _dev(params.gamma_f, dv)
        self.w_head = _dev(params.w_head, dv)
        self._ws: Dict[int, _Workspace] = {}
        self._graphs: Dict[object, object] = {}
        # optional (before, after) callables around every fused scan launch
        # (the bench times that kernel with events on the launch stream)
        self.scan_timer = None
        # row statistics of the rows the last _run left for the head (None: the head reduces them)
        self._head_stats: Optional[torch.Tensor] = None

    # ------------------------------------------------------------ plumbing
    def _workspace(self, T: int) -> _Workspace:
        ws = self._ws.get(T)
        if ws is None:
            ws = _Workspace(self.dims, T, self.device)
            self._ws[T] = ws
        return ws

    def new_state(self, batch: int) -> DecodeState:
        D, N = self.dims.d_inner, self.dims.d_state
        return DecodeState(
            conv=[torch.zeros((batch, 3, D), dtype=torch.int8, device=self.device) for _ in self.layers],
            h=[torch.zeros((batch, D, N), dtype=torch.int32, device=self.device) for _ in self.layers])

    # ---------------------------------------------------------------- layers
    def _layer(self, ly: DeviceLayer, ws: _Workspace, B: int, L: int, conv_state: torch.Tensor,
               h_state: torch.Tensor, fresh: bool, stats_in: Optional[torch.Tensor],
               stats_out: Optional[torch.Tensor]) -> None:
        """A layer over [B, L] tokens (prefill).  stats_in: row statistics of ws.r
        (None: the norm reduces the rows itself); stats_out: zeroed buffer that
        receives the statistics of the updated residual (or None)."""
        dims = self.dims
        D, N, R, d = dims.d_inner, dims.d_state, dims.dt_rank, dims.d_model
        T = B * L
        if dims.ssd:
            self._layer_ssd(ly, ws, B, L, conv_state, h_state, fresh, stats_in, stats_out)
            return
        ops.bitshift_norm(ws.r, ly.gamma, out=ws.a, row_stats=stats_in)
        step = L == 1 and not fresh
        conv_done = not step and self._in_proj_conv_ok()
        if conv_done:
            self._in_proj_conv(ly, ws, B, conv_state, fresh)
        else:
            ops.bitlinear(ws.a, ly.w_in, ops.OUT_INT8, 2 * D, shift=ly.s_in, out=ws.xz)
        if step and self._conv_xproj_ok():
            # one recurrent step per sequence: conv step + x_proj (four blocks per token
            # leaving int32 partials where d_inner allows, else one block per token),
            # then dt_proj + scan step + gate
            if ws.xq is not None:
                ops.conv_step_xpart(ws.xz, D, ly.conv_w, ly.conv_b, conv_state, ly.w_x, dims.xp_width,
                                    xs=ws.xs, xpart=ws.xq)
                ops.xpart_dt_scan_step(ws.xq, ly.s_x, R, ly.w_dt, ly.s_dt, ws.xs, ws.xz, D, ly.base, ly.k,
                                       ly.s_y, h_state, ws.yo)
            else:
                ops.conv_step_xproj(ws.xz, D, ly.conv_w, ly.conv_b, conv_state, ly.w_x, ly.s_x, dims.xp_width,
                                    xs=ws.xs, xp=ws.xp)
                ops.dt_scan_step(ws.xp, R, ly.w_dt, ly.s_dt, ws.xs, ws.xz, D, ly.base, ly.k, ly.s_y, h_state,
                                 ws.yo)
            if self._step_parts(ws):
                # the next norm sums these per-16-feature statistics partials
                ops.bitlinear_residual_parts(ws.yo, ly.w_out, ws.r, ly.res_mult, ly.res_shift, ws.parts,
                                             res_clamp=ly.out_clamp)
            else:
                ops.bitlinear(ws.yo, ly.w_out, ops.OUT_RESIDUAL, d, out=ws.r, res_mult=ly.res_mult,
                              res_shift=ly.res_shift, res_clamp=ly.out_clamp, row_stats=stats_out)
            return
        if not conv_done:
            ops.conv_squareplus(ws.xz, D, ly.conv_w, ly.conv_b, state_in=None if fresh else conv_state,
                                state_out=conv_state, out=ws.xs, batch=B)
        ops.bitlinear(ws.xs, ly.w_x, ops.OUT_INT8, dims.xp_width, shift=ly.s_x, out=ws.xp)
        if step:
            # one recurrent step per sequence (any batch): dt_proj + scan step + gate
            ops.dt_scan_step(ws.xp, R, ly.w_dt, ly.s_dt, ws.xs, ws.xz, D, ly.base, ly.k, ly.s_y, h_state, ws.yo)
            ops.bitlinear(ws.yo, ly.w_out, ops.OUT_RESIDUAL, d, out=ws.r, res_mult=ly.res_mult,
                          res_shift=ly.res_shift, res_clamp=ly.out_clamp, row_stats=stats_out)
            return
        ops.bitlinear(ws.xp, ly.w_dt, ops.OUT_DECAY_MOD, D, k=R, shift=ly.s_dt, out=ws.dm,
                      lda=dims.xp_width, m=T)
        if self.scan_timer is not None:
            self.scan_timer[0]()
        ops.block_scan(ws.xs, ws.dm, ws.xp, R, ws.xz, D, ly.base, ly.k, ly.s_y,
                       h_in=None if fresh else h_state, h_out=h_state, out=ws.yo, batch=B)
        if self.scan_timer is not None:
            self.scan_timer[1]()
        ops.bitlinear(ws.yo, ly.w_out, ops.OUT_RESIDUAL, d, out=ws.r, res_mult=ly.res_mult,
                      res_shift=ly.res_shift, res_clamp=ly.out_clamp, row_stats=stats_out)

    def _layer_ssd(self, ly: DeviceLayer, ws: _Workspace, B: int, L: int, conv_state: torch.Tensor,
                   h_state: torch.Tensor, fresh: bool, stats_in: Optional[torch.Tensor],
                   stats_out: Optional[torch.Tensor]) -> None:
        """A MambaIntegerBlockV2 layer (``ssd_multihead.py:523-592``; spec section 7)
        over [B, L] tokens, prefill or one recurrent step (L = 1)."""
        dims = self.dims
        D, d = dims.d_inner, dims.d_model
        ops.bitshift_norm(ws.r, ly.gamma, out=ws.a, row_stats=stats_in, v2=True)
        if not (L == 1 and not fresh) and self._in_proj_conv_ok():
            self._in_proj_conv(ly, ws, B, conv_state, fresh)
        else:
            ops.bitlinear(ws.a, ly.w_in, ops.OUT_INT8, 2 * D, shift=ly.s_in, out=ws.xz)
            ops.conv_squareplus(ws.xz, D, ly.conv_w, ly.conv_b, state_in=None if fresh else conv_state,
                                state_out=conv_state, out=ws.xs, batch=B)
        ops.bitlinear(ws.xs, ly.w_x, ops.OUT_INT8, dims.xp_width, shift=ly.s_x, out=ws.xp)
        if self.scan_timer is not None:
            self.scan_timer[0]()
        ops.ssd_block_scan(ws.xs, ws.xp, ws.xz, D, ly.decay_tab, dims.n_heads, dims.d_state, ly.s_y,
                           h_in=None if fresh else h_state, h_out=h_state, out=ws.yo, batch=B)
        if self.scan_timer is not None:
            self.scan_timer[1]()
        ops.bitlinear(ws.yo, ly.w_out, ops.OUT_RESIDUAL, d, out=ws.r, res_mult=ly.res_mult,
                      res_shift=ly.res_shift, res_clamp=ly.out_clamp, row_stats=stats_out)

    def _in_proj_conv_ok(self) -> bool:
        """mi_in_proj_conv's limits: d_inner a multiple of 128, d_model of 64."""
        return self.dims.d_inner % 128 == 0 and self.dims.d_model % 64 == 0

    def _in_proj_conv(self, ly: DeviceLayer, ws: _Workspace, B: int, conv_state: torch.Tensor,
                      fresh: bool) -> None:
        """Prefill in_proj with the conv + squareplus of the x half in its epilogue:
        writes ws.xs, the z half of ws.xz and the new conv state.  The old state
        is read from a copy (blocks read a sequence's old state while others
        write its new one)."""
        prev = None if fresh else conv_state.clone()
        ops.in_proj_conv(ws.a, ly.w_in, ly.s_in, self.dims.d_inner, ly.conv_w, ly.conv_b, B, conv_state,
                         state_in=prev, xs=ws.xs, xz=ws.xz)

    def _step_parts(self, ws: _Workspace) -> bool:
        """The batched one-token step (conv step + x_proj kernel) hands the row
        statistics on as out_proj partials (ws.parts), so the norms that follow
        are elementwise instead of reducing their rows."""
        return (self._conv_xproj_ok() and ws.parts is not None and ws.T <= 64
                and self.dims.d_inner % 64 == 0 and not self.dims.ssd)

    def _conv_xproj_ok(self) -> bool:
        """mi_conv_step_xproj's limits (d_inner a multiple of 256 up to 8192,
        x_proj rows <= 256): the batched decode's conv step carries x_proj."""
        D = self.dims.d_inner
        return D % 256 == 0 and D <= 8192 and self.dims.xp_width <= 256

    def _fused_decode_ok(self, B: int) -> bool:
        """The three fused decode stages pay off while the work every block
        repeats stays small: each in_proj block normalizes all B rows of d
        channels, so the repeated work grows as B * d^2.  Measured (ms per step):
        d768 fused wins at every B <= 64 (0.69 vs 0.84 at B64), d1024 at B16 but
        not B64, d1536 and d2048 at no batch."""
        d = self.dims.d_model
        return (B <= 64 and d <= 1024 and B * d * d <= 64 * 768 * 768 and d % 64 == 0 and self.dims.d_state <= 64
                and self.dims.dt_rank <= 256)

    def _layer_decode(self, ly: DeviceLayer, ws: _Workspace, conv_state: torch.Tensor,
                      h_state: torch.Tensor, li: int) -> None:
        """One token per sequence through a layer in three kernels (fused stages).  The
        norm of layer 0 reads the embedding's row statistics (ws.stats[0]), later norms
        and the head the out_proj's per-block partials (ws.parts)."""
        dims = self.dims
        D, R = dims.d_inner, dims.dt_rank
        stats_in = ws.stats[0] if li == 0 else ws.parts
        if dims.ssd:
            # MambaIntegerBlockV2 in four kernels: V2 norm + in_proj + conv step,
            # x_proj, one block-scan step (unit B/C, head decay, gate), out_proj
            ops.norm_in_proj_conv(ws.r, ly.gamma, ly.w_in, ly.s_in, ly.conv_w, ly.conv_b, conv_state, ws.xs, ws.xz,
                                  row_stats=stats_in, v2=True)
            ops.bitlinear(ws.xs, ly.w_x, ops.OUT_INT8, dims.xp_width, shift=ly.s_x, out=ws.xp)
            ops.ssd_block_scan(ws.xs, ws.xp, ws.xz, D, ly.decay_tab, dims.n_heads, dims.d_state, ly.s_y,
                               h_in=h_state, h_out=h_state, out=ws.yo, batch=ws.T)
            ops.bitlinear_residual_parts(ws.yo, ly.w_out, ws.r, ly.res_mult, ly.res_shift, ws.parts,
                                             res_clamp=ly.out_clamp)
            return
        if ws.xpart is not None:
            # x_proj partials from the in_proj blocks, summed by the scan step
            ops.norm_in_proj_conv(ws.r, ly.gamma, ly.w_in, ly.s_in, ly.conv_w, ly.conv_b, conv_state, ws.xs, ws.xz,
                                  row_stats=stats_in, w_x=ly.w_x, xpart=ws.xpart)
            ops.xpart_dt_scan_step(ws.xpart, ly.s_x, R, ly.w_dt, ly.s_dt, ws.xs, ws.xz, D, ly.base, ly.k, ly.s_y,
                                   h_state, ws.yo)
        else:
            ops.norm_in_proj_conv(ws.r, ly.gamma, ly.w_in, ly.s_in, ly.conv_w, ly.conv_b, conv_state, ws.xs, ws.xz,
                                  row_stats=stats_in)
            if dims.xp_width <= 256:
                ops.xproj_dt_scan_step(ws.xs, ly.w_x, ly.s_x, R, ly.w_dt, ly.s_dt, ws.xz, D, ly.base, ly.k, ly.s_y,
                                       h_state, ws.yo)
            else:
                ops.bitlinear(ws.xs, ly.w_x, ops.OUT_INT8, dims.xp_width, shift=ly.s_x, out=ws.xp)
                ops.dt_scan_step(ws.xp, R, ly.w_dt, ly.s_dt, ws.xs, ws.xz, D, ly.base, ly.k, ly.s_y, h_state, ws.yo)
        ops.bitlinear_residual_parts(ws.yo, ly.w_out, ws.r, ly.res_mult, ly.res_shift, ws.parts,
                                             res_clamp=ly.out_clamp)

    def _head(self, r_rows: torch.Tensor, stats: Optional[torch.Tensor],
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Final norm + lm_head (int32 logits).  The fused norm + GEMV pays off only
        with the rows' statistics at hand and few rows: each of its blocks
        normalizes every row (measured, no statistics: B8 d768 10.5 us fused vs
        8.2 us norm + GEMV, B64 d2048 138 vs 26 us)."""
        m, d = r_rows.shape
        if stats is not None and m * d <= 8 * 1024 and d <= 3072 and d % 64 == 0:
            return ops.norm_bitlinear(r_rows, self.gamma_f, self.w_head, ops.OUT_INT32, self.dims.vocab_size,
                                      out=out, row_stats=stats)
        a = ops.bitshift_norm(r_rows, self.gamma_f, row_stats=stats)
        V = self.dims.vocab_size
        if out is not None or V % 4 == 0:
            return ops.bitlinear(a, self.w_head, ops.OUT_INT32, V, out=out)
        # int32 output rows are stored 16 bytes at a time: pad the row stride
        padded = torch.empty((a.shape[0], V + (-V) % 4), dtype=torch.int32, device=a.device)
        ops.bitlinear(a, self.w_head, ops.OUT_INT32, V, out=padded)
        return padded[:, :V].contiguous()

    def _run(self, ids: torch.Tensor, state: DecodeState, fresh: bool) -> _Workspace:
        B, L = ids.shape
        ws = self._workspace(B * L)
        ops.embed(ids.reshape(-1).contiguous(), self.emb, out=ws.r, row_stats=ws.stats[:1])
        decode = L == 1 and not fresh and self._fused_decode_ok(B)
        parts = L == 1 and not fresh and not decode and self._step_parts(ws)
        self._head_stats = ws.parts if decode or parts else None
        for i, ly in enumerate(self.layers):
            if decode:
                self._layer_decode(ly, ws, state.conv[i], state.h[i], i)
            else:
                # prefill: the norm of layer 0 uses the embedding's row statistics; later
                # norms reduce their rows (atomics over 16k-row tiles cost more than they
                # save) or, after a batched one-token step, sum the out_proj's partials
                self._layer(ly, ws, B, L, state.conv[i], state.h[i], fresh,
                            ws.stats[0] if i == 0 else (ws.parts if parts else None), None)
        return ws

    # ------------------------------------------------------------ public API
    @torch.no_grad()
    def forward_logits(self, ids: torch.Tensor) -> torch.Tensor:
        """All-position int32 logits [B, L, V] (MambaIntegerModel.forward)."""
        B, L = ids.shape
        state = self.new_state(B)
        ws = self._run(ids, state, fresh=True)
        return self._head(ws.r, self._head_stats).view(B, L, -1)

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, state: Optional[DecodeState] = None
                ) -> Tuple[torch.Tensor, DecodeState]:
        """Last-position int32 logits [B, V] and the recurrent state after the prompt."""
        B, L = ids.shape
        fresh = state is None
        if state is None:
            state = self.new_state(B)
        ws = self._run(ids, state, fresh=fresh)
        last = ws.r.view(B, L, -1)[:, -1, :].contiguous()
        # statistics only after a one-token step (L == 1): then the last rows are all rows
        return self._head(last, self._head_stats if L == 1 else None), state

    @torch.no_grad()
    def decode_step(self, tokens: torch.Tensor, state: DecodeState) -> torch.Tensor:
        """One recurrent step for tokens [B] int64; updates `state` in place."""
        ws = self._run(tokens.view(-1, 1), state, fresh=False)
        return self._head(ws.r, self._head_stats)

    @torch.no_grad()
    def generate(self, ids: torch.Tensor, n_new: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy decode (first maximal index): returns [B, n_new] int64 token ids."""
        logits, state = self.prefill(ids)
        return self.decode_loop(logits, state, n_new, use_graph=use_graph)

    @torch.no_grad()
    def decode_loop(self, logits: torch.Tensor, state: DecodeState, n_new: int,
                    use_graph: bool = True) -> torch.Tensor:
        """Greedy continuation from last-position logits [B, V] and `state`."""
        B = logits.shape[0]
        out = torch.empty((B, n_new), dtype=torch.int64, device=self.device)
        if n_new == 0:
            return out
        tok = ops.argmax(logits)
        out[:, 0] = tok
        if not use_graph:
            for i in range(1, n_new):
                logits = self.decode_step(tok, state)
                tok = ops.argmax(logits)
                out[:, i] = tok
            return out
        if self._chain_ok(B):
            self._decode_chain_loop(tok, state, out)
            return out
        step = self._decode_graph(B, state)
        step.tok_in.copy_(tok)
        for i in range(1, n_new):
            step.graph.replay()          # embed(tok) ... argmax -> tok
            out[:, i] = step.tok_in
        # hand the state back to the caller's tensors
        for i in range(len(self.layers)):
            state.conv[i].copy_(step.state.conv[i])
            state.h[i].copy_(step.state.h[i])
        return out

    # ------------------------------------------------- multi-step decode graphs
    GRAPH_STEPS = 16

    def _chain_ok(self, B: int) -> bool:
        """The fused chain (three kernels per layer, argmax fused into the head) fits batch B."""
        return self._fused_decode_ok(B)

    def _decode_chain(self, ws: _Workspace, state: DecodeState, hist: torch.Tensor, keys: torch.Tensor) -> None:
        """len(hist) greedy steps.  Step 0 embeds hist[-1] (the previous pick); step j > 0
        picks from step j-1's head keys, writing the pick to hist[j-1], and embeds it;
        the last step's pick goes to hist[-1]."""
        S = hist.shape[0]
        V = self.dims.vocab_size
        for j in range(S):
            if j == 0:
                ops.embed(hist[S - 1], self.emb, out=ws.r, row_stats=ws.stats[:1])
            else:
                ops.embed_argmax(keys, hist[j - 1], self.emb, ws.r, ws.stats[:1])
            for i, ly in enumerate(self.layers):
                self._layer_decode(ly, ws, state.conv[i], state.h[i], i)
            ops.norm_bitlinear_argmax(ws.r, self.gamma_f, self.w_head, V, keys, row_stats=ws.parts)
        ops.argmax_keys(keys, out=hist[S - 1])

    def _chain_graph(self, B: int, S: int):
        """HIP graph of S chained greedy steps for batch B (state, workspace and keys shared
        by every S; hist [S, B] of its own)."""
        g = self._graphs.get((B, S))
        if g is not None:
            return g
        shared = self._graphs.get((B, "shared"))
        if shared is None:
            nk = (self.dims.vocab_size + 63) // 64
            shared = (self.new_state(B), torch.empty((B, nk), dtype=torch.int64, device=self.device))
            self._graphs[(B, "shared")] = shared
        gstate, keys = shared
        ws = self._workspace(B)
        hist = torch.zeros((S, B), dtype=torch.int64, device=self.device)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # one eager pass first: every kernel is loaded before capture
            self._decode_chain(ws, gstate, hist, keys)
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                self._decode_chain(ws, gstate, hist, keys)
        torch.cuda.current_stream().wait_stream(side)
        g = (graph, hist, gstate)
        self._graphs[(B, S)] = g
        return g

    def _decode_chain_loop(self, tok: torch.Tensor, state: DecodeState, out: torch.Tensor) -> None:
        """Fills out[:, 1:] by replaying chain graphs of GRAPH_STEPS steps (and one of the
        remainder), starting from pick `tok` and `state`; the state is handed back."""
        B, n_new = out.shape
        if n_new <= 1:
            return
        # every graph this run replays is captured first: capture runs an eager
        # pass over the shared graph state, which must not happen mid-run
        sizes = [min(self.GRAPH_STEPS, n_new - i) for i in range(1, n_new, self.GRAPH_STEPS)]
        for S in set(sizes):
            self._chain_graph(B, S)
        gstate = self._chain_graph(B, sizes[0])[2]
        for li in range(len(self.layers)):
            gstate.conv[li].copy_(state.conv[li])
            gstate.h[li].copy_(state.h[li])
        i = 1
        prev = tok
        for S in sizes:
            graph, hist, _ = self._chain_graph(B, S)
            if prev.data_ptr() != hist[S - 1].data_ptr():
                hist[S - 1].copy_(prev)
            graph.replay()
            out[:, i:i + S] = hist.t()
            prev = hist[S - 1]
            i += S
        for li in range(len(self.layers)):
            state.conv[li].copy_(gstate.conv[li])
            state.h[li].copy_(gstate.h[li])

    def _decode_body(self, ws: _Workspace, state: DecodeState, tok: torch.Tensor, logits: torch.Tensor,
                     tok_out: torch.Tensor) -> None:
        """embed -> layers -> head -> argmax for one token per sequence (graph body)."""
        B = tok.shape[0]
        fused = self._fused_decode_ok(B)
        # the fused layers hand row statistics on as out_proj partials
        ops.embed(tok, self.emb, out=ws.r, row_stats=ws.stats[:1])
        parts = not fused and self._step_parts(ws)
        for i, ly in enumerate(self.layers):
            if fused:
                self._layer_decode(ly, ws, state.conv[i], state.h[i], i)
            else:
                # the batched layers' norms sum the previous out_proj's statistics
                # partials, or reduce their rows where the step cannot store them
                self._layer(ly, ws, B, 1, state.conv[i], state.h[i], False,
                            ws.stats[0] if i == 0 else (ws.parts if parts else None), None)
        self._head(ws.r, ws.parts if fused or parts else None, out=logits)
        ops.argmax(logits, out=tok_out)

    def _decode_graph(self, B: int, state: DecodeState):
        """Captures embed -> layers -> head -> argmax for batch B as one HIP graph."""
        g = self._graphs.get(B)
        if g is None:
            tok_in = torch.zeros((B,), dtype=torch.int64, device=self.device)  # read by embed, rewritten by argmax
            gstate = self.new_state(B)
            # warm the workspaces outside capture (allocation happens here)
            ws = self._workspace(B)
            logits = torch.empty((B, self.dims.vocab_size), dtype=torch.int32, device=self.device)
            tok_out = tok_in
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                # one eager step first: every kernel is loaded before capture
                self._decode_body(ws, gstate, tok_in, logits, tok_out)
                tok_in.zero_()
            side.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(graph, stream=side):
                    self._decode_body(ws, gstate, tok_in, logits, tok_out)
            torch.cuda.current_stream().wait_stream(side)

            class _G:
                pass
            g = _G()
            g.graph, g.tok_in, g.tok_out, g.state = graph, tok_in, tok_out, gstate
            self._graphs[B] = g
        for i in range(len(self.layers)):
            g.state.conv[i].copy_(state.conv[i])
            g.state.h[i].copy_(state.h[i])
        return g
