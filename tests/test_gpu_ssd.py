"""GPU parity of the multi-head SSD block (MambaIntegerBlockV2, spec section 7)
against the oracle: the V2 norm, the block scan (prefill chunks, ragged
lengths, state in/out, one-step decode) and the whole model (prefill logits,
greedy decode, the drop-in module)."""
import numpy as np
import pytest

import oracle as O
from mamba_int import ModelDims, init_random_params, ssd_decay_table

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("rows,d", [(5, 768), (300, 256), (7, 96)])
def test_norm_v2(cuda, rows, d):
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(rows + d)
    r = rng.integers(-(2**23) + 1, 2**23, size=(rows, d), dtype=np.int32)
    r[0] >>= 12
    r[1] >>= 20
    g = rng.integers(-400, 400, size=d, dtype=np.int16)
    ref = O.bitshift_norm_v2(r, g)
    assert np.array_equal(H(ops.bitshift_norm(T(r), T(g), v2=True)), ref)
    if d % 4 == 0:
        r64 = r.astype(np.int64)
        st = T(np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
        assert np.array_equal(H(ops.bitshift_norm(T(r), T(g), row_stats=st, v2=True)), ref)


def _inputs(rng, B, L, Hh, P, N, tab_kind):
    D = Hh * P
    W = -(-(2 * Hh * N + Hh) // 16) * 16
    xs = rng.integers(-127, 128, size=(B, L, D)).astype(np.int8)
    xp = rng.integers(-127, 128, size=(B, L, W)).astype(np.int8)
    xz = rng.integers(-127, 128, size=(B, L, 2 * D)).astype(np.int8)
    if tab_kind == "model":
        tab = ssd_decay_table(rng.uniform(-2.3, -0.01, size=Hh))
    else:
        tab = rng.integers(0, 32769, size=(Hh, 255)).astype(np.int32)
    h0 = rng.integers(-(2**26), 2**26, size=(B, D, N)).astype(np.int32)
    return xs, xp, xz, tab, h0


@pytest.mark.parametrize("B,L,Hh,P,N,tab_kind", [
    (2, 100, 3, 32, 16, "model"), (1, 64, 2, 64, 64, "model"), (3, 5, 4, 16, 32, "random"),
    (2, 130, 24, 64, 64, "model"), (1, 1, 2, 64, 64, "random"), (4, 67, 2, 48, 16, "random"),
])
def test_ssd_block_scan(cuda, B, L, Hh, P, N, tab_kind):
    """mi_ssd_block_scan equals the oracle from a zero state and from a given
    state (final states too), over chunk-ragged lengths and every N."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(B * 1000 + L + Hh + P + N)
    xs, xp, xz, tab, h0 = _inputs(rng, B, L, Hh, P, N, tab_kind)
    D = Hh * P
    for start in (None, h0):
        ref_y, ref_h = O.ssd_v2_scan(xs, xp, xz, D, tab, 14, Hh, N, h_state=start)
        hs = T(start) if start is not None else None
        hout = torch.zeros((B, D, N), dtype=torch.int32, device="cuda")
        yo = ops.ssd_block_scan(T(xs), T(xp), T(xz), D, T(tab), Hh, N, 14, h_in=hs, h_out=hout)
        assert np.array_equal(H(yo), ref_y)
        assert np.array_equal(H(hout), ref_h)


def test_ssd_block_scan_decode_steps(cuda):
    """Step-by-step (L = 1, state in place) equals one pass over the sequence."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(4)
    B, L, Hh, P, N = 3, 9, 4, 32, 32
    xs, xp, xz, tab, _ = _inputs(rng, B, L, Hh, P, N, "model")
    D = Hh * P
    ref_y, ref_h = O.ssd_v2_scan(xs, xp, xz, D, tab, 13, Hh, N)
    h = torch.zeros((B, D, N), dtype=torch.int32, device="cuda")
    ys = []
    for t in range(L):
        ys.append(H(ops.ssd_block_scan(T(xs[:, t:t + 1]), T(xp[:, t:t + 1]), T(xz[:, t:t + 1]), D, T(tab), Hh, N,
                                       13, h_in=h, h_out=h)))
    assert np.array_equal(np.concatenate(ys, 1), ref_y)
    assert np.array_equal(H(h), ref_h)


@pytest.mark.parametrize("P", [16, 32, 64])
@pytest.mark.parametrize("N", [16, 32, 64])
def test_ssd_one_step_kernel(cuda, P, N):
    """The one-step form of the SSD block scan (len 1: a block per sequence and
    head) from a random state in place and from no state, every (d_head,
    d_state) it takes, against the oracle."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(P * 7 + N)
    B, Hh = 5, 3
    xs, xp, xz, tab, _ = _inputs(rng, B, 1, Hh, P, N, "random" if N == 32 else "model")
    D = Hh * P
    h0 = rng.integers(-(2**25), 2**25, size=(B, D, N), dtype=np.int32)
    ref_y, ref_h = O.ssd_v2_scan(xs, xp, xz, D, tab, 12, Hh, N, h_state=h0)
    h = T(h0)
    y = ops.ssd_block_scan(T(xs), T(xp), T(xz), D, T(tab), Hh, N, 12, h_in=h, h_out=h)
    assert np.array_equal(H(y), ref_y) and np.array_equal(H(h), ref_h)
    ref_y0, ref_h0 = O.ssd_v2_scan(xs, xp, xz, D, tab, 12, Hh, N)
    h1 = torch.full((B, D, N), 3, dtype=torch.int32, device="cuda")
    y0 = ops.ssd_block_scan(T(xs), T(xp), T(xz), D, T(tab), Hh, N, 12, h_out=h1)
    assert np.array_equal(H(y0), ref_y0) and np.array_equal(H(h1), ref_h0)


def _ssd_params(seed=11, d=128, n_layer=2, V=400, N=16, Hh=4, P=64):
    dims = ModelDims(d_model=d, n_layer=n_layer, vocab_size=V, d_state=N, dt_rank=0, block="ssd", n_heads=Hh,
                     d_head=P)
    return init_random_params(dims, seed)


@pytest.mark.parametrize("N,Hh,P", [(16, 4, 64), (64, 2, 128)])
def test_ssd_model_prefill_and_decode(cuda, N, Hh, P):
    """Prefill logits at every position and greedy decode (eager steps and the
    captured step graph) equal the oracle's."""
    from mamba_int.model import IntegerMambaRunner
    p = _ssd_params(N=N, Hh=Hh, P=P)
    om = O.OracleModel(p)
    ids = np.random.default_rng(3).integers(0, 400, size=(2, 21))
    run = IntegerMambaRunner(p)
    assert np.array_equal(H(run.forward_logits(T(ids))), om.forward(ids))
    ref = om.generate(ids, 7)
    assert np.array_equal(H(run.generate(T(ids), 7, use_graph=False)), ref)
    assert np.array_equal(H(run.generate(T(ids), 7, use_graph=True)), ref)


def test_ssd_dropin_model(cuda):
    """MambaIntegerModel with ssm_cfg.use_ssd (the shipped config's block choice,
    mamba_integer_model.py:473-476) builds multi-head SSD layers and matches the
    oracle; MambaIntegerBlockV2 alone updates the residual like the model's layer."""
    import torch
    from mamba_integer_model import MambaIntegerBlockV2, MambaIntegerModel
    cfg = {"d_model": 128, "n_layer": 2, "vocab_size": 300,
           "ssm_cfg": {"d_state": 32, "use_ssd": True, "n_heads": 4, "d_head": 64}}
    model = MambaIntegerModel(cfg, seed=2)
    assert model.dims.ssd and model.dims.d_inner == 256
    ids = np.random.default_rng(6).integers(0, 300, size=(2, 9))
    om = O.OracleModel(model.params)
    assert np.array_equal(H(model.forward_int(T(ids))), om.forward(ids))
    blk = MambaIntegerBlockV2(cfg, 0, params=model.params.layers[0])
    r0 = O.embed(ids.reshape(-1), model.params.emb)
    got = blk(T(r0.reshape(2, 9, 128)))
    want, _ = om._layer_ssd(model.params.layers[0], r0, 2, 9, None)
    assert np.array_equal(H(got).reshape(-1, 128), want)
    torch.cuda.synchronize()
