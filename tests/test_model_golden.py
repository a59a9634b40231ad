"""Whole-model golden fixtures (tests/golden/model_*_small.npz).

make_golden.py states the model's composition a second time, in Python
integers, from the reference forward passes (MambaIntegerModel.forward,
mamba_integer_model.py:486-495; MambaIntegerBlock.forward, :396-447;
MambaIntegerBlockV2.forward, ssd_multihead.py:523-592), and generates by
recomputing the whole prefix per token (scripts/inference.py:147-161).  These
tests hold the oracle's OracleModel, the GPU runner and the native decode step
to those vectors: all-position logits of two 12-token prompts and 8 greedy
tokens each, for 2-layer models of each block type: "small" ones whose greedy
tokens vary and depend on the history, and "wide" ones whose residual
updates saturate and whose final norm runs past the top of the BitShiftNormV2
table.  In both SSD fixtures the block's out_proj clamp (ssd_multihead.py:
589-590) binds on a hundred-odd accumulators of the stored logits.  Planted
wiring mistakes in OracleModel must fail them.
"""
import os

import numpy as np
import pytest

import oracle as O
from mamba_int import ModelDims
from mamba_int.params import LayerParams, ModelParams, SSDLayerParams, ssd_decay_table

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["model_dyadic_small.npz", "model_ssd_small.npz", "model_dyadic_wide.npz", "model_ssd_wide.npz"]


def load(name):
    """The fixture's arrays and its integer model as ModelParams."""
    with np.load(os.path.join(GOLDEN, name)) as f:
        g = {k: f[k] for k in f.files}
    ssd = "l0_decay_tab" in g
    V, d = g["emb"].shape
    names = [str(s) for s in g["scalar_names"]]
    layers = []
    nl = sum(1 for k in g if k.endswith("_scalars"))
    for i in range(nl):
        sc = dict(zip(names, (int(v) for v in g[f"l{i}_scalars"])))
        common = dict(gamma=g[f"l{i}_gamma"], w_in=g[f"l{i}_w_in_packed"], s_in=sc["s_in"],
                      conv_w=g[f"l{i}_conv_w"], conv_b=g[f"l{i}_conv_b"], w_x=g[f"l{i}_w_x_packed"],
                      s_x=sc["s_x"], s_y=sc["s_y"], w_out=g[f"l{i}_w_out_packed"], res_mult=sc["res_mult"],
                      res_shift=sc["res_shift"])
        if ssd:
            layers.append(SSDLayerParams(decay_tab=g[f"l{i}_decay_tab"], out_clamp=sc["out_clamp"], **common))
        else:
            layers.append(LayerParams(w_dt=g[f"l{i}_w_dt_packed"], s_dt=sc["s_dt"], base=g[f"l{i}_base"], k=15,
                                      **common))
    if ssd:
        H = g["l0_decay_tab"].shape[0]
        D = g["l0_conv_b"].shape[0]
        dims = ModelDims(d_model=d, n_layer=nl, vocab_size=V, d_state=16, dt_rank=0, block="ssd", n_heads=H,
                         d_head=D // H)
    else:
        R = g["l0_w_dt"].shape[1]
        N = g["l0_base"].shape[1]
        dims = ModelDims(d_model=d, n_layer=nl, vocab_size=V, d_state=N, dt_rank=R)
    p = ModelParams(dims=dims, emb=g["emb"], layers=layers, gamma_f=g["gamma_f"], w_head=g["w_head_packed"])
    return g, p


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_packing_matches_the_product_packer(name):
    """The fixture's own pure-Python packing agrees with mamba_int.pack_ternary."""
    from mamba_int import pack_ternary
    g, _ = load(name)
    for k in g:
        if k.endswith("_packed"):
            assert np.array_equal(pack_ternary(g[k[:-len("_packed")]]), g[k]), k


def test_ssd_decay_table_matches_python_math():
    """params.ssd_decay_table (numpy float64) equals the fixture's statement in
    Python's math module on every entry."""
    g, _ = load("model_ssd_small.npz")
    for i in range(2):
        assert np.array_equal(ssd_decay_table(g[f"l{i}_a_log"]), g[f"l{i}_decay_tab"])


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_model_matches_whole_model_fixture(name):
    g, p = load(name)
    om = O.OracleModel(p)
    assert np.array_equal(om.forward(g["ids"]), g["logits"])
    assert np.array_equal(om.generate(g["ids"], g["gen"].shape[1]), g["gen"])


@pytest.mark.parametrize("name,mutation", [
    (f"model_{blk}_{kind}.npz", m) for kind in ("small", "wide") for blk in ("dyadic", "ssd")
    for m in ("swap_xz", "norm_f_v2", "no_residual") + (("block_norm_v1", "no_out_clamp") if blk == "ssd" else ())
] + [("model_dyadic_small.npz", "conv_reset"), ("model_ssd_small.npz", "conv_reset")])
def test_wiring_mutations_are_caught(name, mutation):
    """Each planted wiring mistake in OracleModel changes the logits or the
    greedy tokens away from the fixture (conv_reset only touches the recurrent
    step, so only the tokens can show it)."""
    g, p = load(name)
    O.set_wiring_mutation(mutation)
    try:
        om = O.OracleModel(p)
        same_logits = np.array_equal(om.forward(g["ids"]), g["logits"])
        same_gen = np.array_equal(om.generate(g["ids"], g["gen"].shape[1]), g["gen"])
    finally:
        O.set_wiring_mutation(None)
    assert not (same_logits and same_gen), mutation
    if mutation == "conv_reset":
        assert same_logits and not same_gen


# ------------------------------------------------------------------ GPU
def _T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_gpu_runner_matches_whole_model_fixture(cuda, name):
    """IntegerMambaRunner: all-position logits, and greedy generation eager,
    through the single-step graph and through the chained graphs."""
    from mamba_int.model import IntegerMambaRunner
    g, p = load(name)
    run = IntegerMambaRunner(p)
    ids = _T(g["ids"])
    assert np.array_equal(run.forward_logits(ids).cpu().numpy(), g["logits"])
    n = g["gen"].shape[1]
    assert np.array_equal(run.generate(ids, n, use_graph=False).cpu().numpy(), g["gen"])
    assert np.array_equal(run.generate(ids, n, use_graph=True).cpu().numpy(), g["gen"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_gpu_native_decode_step_matches_whole_model_fixture(cuda, name):
    """mi_decode_step (the whole greedy step behind the C ABI) continues the
    runner's prefill to the fixture's tokens."""
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    g, p = load(name)
    run = IntegerMambaRunner(p)
    logits, st = run.prefill(_T(g["ids"]))
    first = ops.argmax(logits)
    got = NativeDecoder(run, g["ids"].shape[0]).generate(first, st, g["gen"].shape[1])
    assert np.array_equal(got.cpu().numpy(), g["gen"])
