"""GPU parity at the full benchmark workloads.

Batch lanes are independent in every kernel of the stack (each sequence has
its own rows, conv ring and scan state), so the oracle runs a few of a batch's
sequences on their own and the GPU result for those rows must match it bit
for bit:

- the fused prefill block scan at the config-3 shape (B8, L2048, d_inner 1536,
  N16): the whole batch, with the state carried across the length;
- config 3 (d768 x 24, vocab 32000): batch 8 x 2048-token prefill, then 256
  greedy steps through the chained decode graphs, as the benchmark runs it;
  two of the eight sequences against the oracle;
- config 5 (d2048 x 48, d_inner 4096, vocab 32000): batch 64 x 512-token
  prefill, then 1024 greedy steps through the batched decode path; one
  sequence against the oracle over 256 steps, and for the whole batch the
  decode logits after the 1024th step against a prefill of the extended
  prompts.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


def _host_params(p):
    """ModelParams with device tensors -> the same with numpy arrays."""
    import dataclasses
    from mamba_int.params import ModelParams

    def conv(v):
        return v.cpu().numpy() if hasattr(v, "cpu") else v
    layers = [dataclasses.replace(lp, **{f.name: conv(getattr(lp, f.name)) for f in dataclasses.fields(lp)})
              for lp in p.layers]
    return ModelParams(dims=p.dims, emb=conv(p.emb), layers=layers, gamma_f=conv(p.gamma_f), w_head=conv(p.w_head))


def _oracle_greedy(om, ids, n_new):
    """Prefill logits, n_new greedy tokens, and the logits after the last one."""
    lg, st = om.prefill(ids)
    first = lg
    toks = []
    for i in range(n_new):
        tok = np.argmax(lg, axis=-1)
        toks.append(tok)
        lg, st = om.decode_step(tok, st)
    return first, np.stack(toks, axis=1), lg


def test_block_scan_config3_shape(cuda):
    """model_scan_kernel at B8 x L2048, d_inner 1536, N16 (the benchmark's
    prefill scan, state carried over all 2048 steps) against the oracle."""
    from mamba_int import ops
    rng = np.random.default_rng(2048)
    B, L, D, N, R = 8, 2048, 1536, 16, 48
    W = R + 2 * N
    xs = rng.integers(0, 128, size=(B, L, D), dtype=np.int8)
    dm = rng.integers(-20, 21, size=(B, L, D), dtype=np.int8)
    xp = rng.integers(-127, 128, size=(B, L, W), dtype=np.int8)
    z = rng.integers(-127, 128, size=(B, L, 2 * D), dtype=np.int8)
    base = rng.integers(16384, 32001, size=(D, N), dtype=np.int32)
    yo_ref, h_ref = O.block_scan(xs, dm, xp, R, z, D, base, 15, 14)
    h = T(np.zeros((B, D, N), np.int32))
    yo = ops.block_scan(T(xs), T(dm), T(xp), R, T(z), D, T(base), 15, 14, h_out=h)
    assert np.array_equal(H(yo), yo_ref)
    assert np.array_equal(H(h), h_ref)


def test_config3_workload(cuda):
    """Config 3 exactly as the benchmark runs it: the same random model (seed 3)
    and prompts, batch 8 x 2048 prefill, 256 greedy decode steps through the
    chained HIP graphs (state handed back), then one more step; sequences 0
    and 5 against the oracle: prefill logits, all 256 tokens, final logits."""
    from mamba_int import ModelDims, init_random_params
    from mamba_int.model import IntegerMambaRunner
    dims = ModelDims(d_model=768, n_layer=24, vocab_size=32000, d_state=16, dt_rank=48)
    p = init_random_params(dims, 3)
    ids = np.random.default_rng(3).integers(0, dims.vocab_size, size=(8, 2048))
    run = IntegerMambaRunner(p)
    lg, st = run.prefill(T(ids))
    lg0 = H(lg)
    gen = run.decode_loop(lg, st, 256, use_graph=True)
    final = H(run.decode_step(gen[:, -1].contiguous(), st))
    gen = H(gen)
    sel = [0, 5]
    ref_lg0, ref_gen, ref_final = _oracle_greedy(O.OracleModel(p), ids[sel], 256)
    assert np.array_equal(lg0[sel], ref_lg0)
    assert np.array_equal(gen[sel], ref_gen)
    assert np.array_equal(final[sel], ref_final)


def test_config5_workload(cuda):
    """Config 5 as the benchmark defines it: batch 64 x 512 prefill and 1024
    greedy steps through the batched decode path (chained HIP graphs).
    Sequence 37 against the oracle over the first 256 steps: prefill logits,
    the 256 tokens and the logits after the 256th.  For the whole batch, the
    decode logits after the 1024th token equal the prefill logits of the 64
    prompts extended by all their generated tokens (1536 positions)."""
    import torch
    from mamba_int import ModelDims
    from mamba_int.model import IntegerMambaRunner, random_device_params
    dims = ModelDims(d_model=2048, n_layer=48, vocab_size=32000, d_state=16, dt_rank=128)
    pd = random_device_params(dims, 5, "cuda:0")
    run = IntegerMambaRunner(pd)
    ids = np.random.default_rng(5).integers(0, dims.vocab_size, size=(64, 512))
    n_ref, n_new = 256, 1024
    lg, st = run.prefill(T(ids))
    lg0 = H(lg)
    gen1 = run.decode_loop(lg, st, n_ref, use_graph=True)
    lg_ref = run.decode_step(gen1[:, -1].contiguous(), st)
    lg_ref_h = H(lg_ref)
    gen2 = run.decode_loop(lg_ref, st, n_new - n_ref, use_graph=True)
    final = run.decode_step(gen2[:, -1].contiguous(), st)
    ext = torch.cat([T(ids), gen1, gen2], dim=1)
    assert ext.shape == (64, 512 + n_new)
    lg_ext, _ = run.prefill(ext)
    assert torch.equal(lg_ext, final)
    gen1 = H(gen1)
    del st, lg_ext, ext, final, gen2
    sel = [37]
    ref_lg0, ref_gen, ref_lg = _oracle_greedy(O.OracleModel(_host_params(pd)), ids[sel], n_ref)
    assert np.array_equal(lg0[sel], ref_lg0)
    assert np.array_equal(gen1[sel], ref_gen)
    assert np.array_equal(lg_ref_h[sel], ref_lg)
