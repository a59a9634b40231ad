"""GPU parity of the full integer Mamba stack against the CPU oracle."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


def _small():
    from mamba_int import ModelDims, init_random_params
    dims = ModelDims(d_model=128, n_layer=3, vocab_size=500, d_state=16, dt_rank=16)
    return init_random_params(dims, 21)


def test_model_forward_logits(cuda):
    from mamba_int.model import IntegerMambaRunner
    p = _small()
    ids = np.random.default_rng(0).integers(0, 500, size=(2, 70))
    ref = O.OracleModel(p).forward(ids)
    got = H(IntegerMambaRunner(p).forward_logits(T(ids)))
    assert np.array_equal(got, ref)


def test_model_prefill_decode_and_generate(cuda):
    from mamba_int.model import IntegerMambaRunner
    p = _small()
    ids = np.random.default_rng(1).integers(0, 500, size=(3, 40))
    om = O.OracleModel(p)
    run = IntegerMambaRunner(p)
    lg_ref, st_ref = om.prefill(ids)
    lg, st = run.prefill(T(ids))
    assert np.array_equal(H(lg), lg_ref)
    for i in range(3):
        assert np.array_equal(H(st.conv[i]), st_ref[i].conv)
        assert np.array_equal(H(st.h[i]), st_ref[i].h)
    gen_ref = om.generate(ids, 6)
    assert np.array_equal(H(run.generate(T(ids), 6, use_graph=False)), gen_ref)
    assert np.array_equal(H(run.generate(T(ids), 6, use_graph=True)), gen_ref)


def test_decode_equals_prefill_at_every_position(cuda):
    """Invariant: step-decode logits at position t equal prefill logits at t."""
    from mamba_int.model import IntegerMambaRunner
    p = _small()
    ids = np.random.default_rng(2).integers(0, 500, size=(2, 24))
    run = IntegerMambaRunner(p)
    full = H(run.forward_logits(T(ids)))
    lg, st = run.prefill(T(ids[:, :5]))
    assert np.array_equal(H(lg), full[:, 4])
    for t in range(5, 24):
        lg = run.decode_step(T(ids[:, t]), st)
        assert np.array_equal(H(lg), full[:, t])


def test_graph_replays_match_eager(cuda):
    """The captured decode graph, replayed many times with eager work between
    replays, gives the eager result every time."""
    from mamba_int.model import IntegerMambaRunner
    p = _small()
    ids = np.random.default_rng(3).integers(0, 500, size=(4, 16))
    run = IntegerMambaRunner(p)
    eager = H(run.generate(T(ids), 12, use_graph=False))
    for _ in range(3):
        assert np.array_equal(H(run.generate(T(ids), 12, use_graph=True)), eager)
        run.forward_logits(T(ids))


def test_config3_width_model_one_sequence(cuda):
    """Config-3 architecture (d768 x 24, d_inner 1536, N16, vocab 32000) on one
    64-token sequence + 4 decode steps, bit-exact with the oracle."""
    from mamba_int import ModelDims, init_random_params
    from mamba_int.model import IntegerMambaRunner
    dims = ModelDims(d_model=768, n_layer=24, vocab_size=32000, d_state=16, dt_rank=48)
    p = init_random_params(dims, 3)
    ids = np.random.default_rng(3).integers(0, 32000, size=(1, 64))
    run = IntegerMambaRunner(p)
    om = O.OracleModel(p)
    lg_ref, _ = om.prefill(ids)
    lg, _ = run.prefill(T(ids))
    assert np.array_equal(H(lg), lg_ref)
    assert np.array_equal(H(run.generate(T(ids), 4, use_graph=True)), om.generate(ids, 4))


def test_dropin_model_api(cuda):
    import torch
    from mamba_integer_model import MambaIntegerModel
    cfg = {"d_model": 128, "n_layer": 2, "vocab_size": 300, "ssm_cfg": {"d_state": 16, "dt_rank": 16}}
    m = MambaIntegerModel(cfg, seed=5)
    ids = torch.randint(0, 300, (2, 20)).cuda()
    logits = m(ids)
    assert logits.shape == (2, 20, 300) and logits.dtype == torch.float32
    ref = O.OracleModel(m.params).forward(ids.cpu().numpy())
    assert np.array_equal(H(m.forward_int(ids)), ref)
    out = m.generate(ids, 5)
    assert out.shape == (2, 25)
    assert np.array_equal(H(out[:, 20:]), O.OracleModel(m.params).generate(ids.cpu().numpy(), 5))


def test_chained_decode_graphs_long_generation(cuda):
    """Greedy generation through the chained multi-step graphs (16 steps per
    replay, argmax fused into the head, a remainder graph) equals the oracle's,
    and the state handed back continues the sequence exactly."""
    from mamba_int.model import IntegerMambaRunner
    p = _small()
    ids = np.random.default_rng(4).integers(0, 500, size=(3, 12))
    om = O.OracleModel(p)
    run = IntegerMambaRunner(p)
    ref = om.generate(ids, 40)
    got = H(run.generate(T(ids), 40, use_graph=True))
    assert np.array_equal(got, ref)
    assert np.array_equal(H(run.generate(T(ids), 40, use_graph=True)), ref)
    # state continuity: 20 + 20 steps through decode_loop equals 40 in one go
    lg, st = run.prefill(T(ids))
    first = H(run.decode_loop(lg, st, 20))
    lg2 = run.decode_step(T(first[:, -1]), st)
    second = H(run.decode_loop(lg2, st, 20))
    assert np.array_equal(np.concatenate([first, second], 1), ref)


def test_config5_width_model_batch64_decode(cuda):
    """Config-5 architecture (d2048, d_inner 4096, N16, dt_rank 128, vocab
    32000) with 2 layers at batch 64: prefill + recurrent decode through the
    batched path (above the fused stages' 16-token limit), bit-exact."""
    from mamba_int import ModelDims, init_random_params
    from mamba_int.model import IntegerMambaRunner
    dims = ModelDims(d_model=2048, n_layer=2, vocab_size=32000, d_state=16, dt_rank=128)
    p = init_random_params(dims, 5)
    ids = np.random.default_rng(6).integers(0, 32000, size=(64, 6))
    ref = O.OracleModel(p).generate(ids, 3)
    run = IntegerMambaRunner(p)
    assert np.array_equal(H(run.generate(T(ids), 3, use_graph=False)), ref)
    assert np.array_equal(H(run.generate(T(ids), 3, use_graph=True)), ref)
    # the native step takes its batched stages here (d_model 2048)
    from mamba_int import ops
    from mamba_int.native import NativeDecoder
    import torch
    lg, st = run.prefill(T(ids))
    dec = NativeDecoder(run, 64)
    assert np.array_equal(H(dec.generate(ops.argmax(lg), st, 3)), ref)
    # its logits at an odd row stride equal the runner's step
    lg, st = run.prefill(T(ids))
    st2 = st.clone()
    tok = ops.argmax(lg)
    buf = torch.zeros((64, 32001), dtype=torch.int32, device="cuda")
    nxt = torch.empty_like(tok)
    dec.step(tok, st, nxt, logits=buf[:, :32000])
    ref_logits = run.decode_step(tok, st2)
    assert np.array_equal(H(buf[:, :32000]), H(ref_logits))
    assert np.array_equal(H(nxt), H(ops.argmax(ref_logits)))


@pytest.mark.parametrize("B", [40, 64])
def test_fused_decode_row_groups(cuda, B):
    """Above 16 sequences the fused decode stages run 16-token row groups in
    one launch (blockIdx.y): greedy continuation (eager and chained graphs) and
    the native step equal the oracle."""
    from mamba_int import ModelDims, init_random_params, ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    dims = ModelDims(d_model=256, n_layer=2, vocab_size=700, d_state=16, dt_rank=16)
    p = init_random_params(dims, 23)
    ids = np.random.default_rng(B).integers(0, 700, size=(B, 5))
    ref = O.OracleModel(p).generate(ids, 6)
    run = IntegerMambaRunner(p)
    assert run._fused_decode_ok(B)
    assert np.array_equal(H(run.generate(T(ids), 6, use_graph=False)), ref)
    assert np.array_equal(H(run.generate(T(ids), 6, use_graph=True)), ref)
    lg, st = run.prefill(T(ids))
    assert np.array_equal(H(NativeDecoder(run, B).generate(ops.argmax(lg), st, 6)), ref)


def test_native_decode_step_matches_oracle(cuda):
    """mi_decode_step (the whole step behind the C ABI): greedy continuation
    equals the oracle's, its logits equal the runner's decode_step logits, and
    a HIP graph of the step replays to the eager result."""
    import torch
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    p = _small()
    ids = np.random.default_rng(8).integers(0, 500, size=(3, 12))
    ref = O.OracleModel(p).generate(ids, 10)
    run = IntegerMambaRunner(p)
    lg, st = run.prefill(T(ids))
    first = ops.argmax(lg)
    dec = NativeDecoder(run, 3)
    assert np.array_equal(H(dec.generate(first, st, 10)), ref)
    # logits: native step vs the runner's staged decode_step on equal states
    lg, st = run.prefill(T(ids))
    st2 = st.clone()
    tok = ops.argmax(lg)
    logits = torch.zeros((3, 500), dtype=torch.int32, device="cuda")
    nxt = torch.empty_like(tok)
    dec.step(tok, st, nxt, logits=logits)
    ref_logits = run.decode_step(tok, st2)
    assert np.array_equal(H(logits), H(ref_logits))
    assert np.array_equal(H(nxt), H(ops.argmax(ref_logits)))
    # graph capture of the native step, replayed with eager work in between
    lg, st = run.prefill(T(ids))
    tok = ops.argmax(lg)
    eager = H(dec.generate(tok, st.clone(), 6))
    cur = tok.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            dec.step(cur, st, nxt)
    torch.cuda.current_stream().wait_stream(side)
    got = [H(cur)]
    for _ in range(5):
        g.replay()
        cur.copy_(nxt)
        got.append(H(cur))
        run.forward_logits(T(ids[:, :4]))  # unrelated eager work between replays
    assert np.array_equal(np.stack(got, 1), eager)


@pytest.mark.parametrize("block", ["dyadic", "ssd"])
def test_chunked_prefill_equals_one_prefill(cuda, block):
    """Prefill continued from a carried state (the fused in_proj + conv reads
    the previous conv state; chunks of 5, 2, 1 and 16 tokens, the short ones
    shorter than the conv window) gives the logits and the conv and scan
    states of one prefill over the whole prompt, and of the oracle."""
    from mamba_int.model import IntegerMambaRunner
    if block == "ssd":
        from test_gpu_ssd import _ssd_params
        p = _ssd_params()
        V = 400
    else:
        p = _small()
        V = 500
    ids = np.random.default_rng(9).integers(0, V, size=(3, 24))
    run = IntegerMambaRunner(p)
    lg_all, st_all = run.prefill(T(ids))
    st = None
    t = 0
    for n in (5, 2, 1, 16):
        lg, st = run.prefill(T(ids[:, t:t + n]), st)
        t += n
    assert np.array_equal(H(lg), H(lg_all))
    for a, b in zip(st.conv + st.h, st_all.conv + st_all.h):
        assert np.array_equal(H(a), H(b))
    assert np.array_equal(H(lg_all), O.OracleModel(p).prefill(ids)[0])
