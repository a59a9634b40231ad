"""mi_decode_step_static: the whole greedy decode step with the library's
static device workspace (no allocation), against mi_decode_step with a
caller-owned workspace, bit for bit, through the C ABI: eager calls in a row,
calls captured in a graph and replayed, and the refusal of a call that would
overlap the previous one on another stream."""
import ctypes

import numpy as np
import pytest


def _model(d_model, n_layer, vocab):
    from mamba_int import ModelDims, init_random_params
    dims = ModelDims(d_model=d_model, n_layer=n_layer, vocab_size=vocab, d_state=16, dt_rank=max(16, d_model // 16))
    return init_random_params(dims, 17)


def _static_step(dec, ids, state, next_ids, logits):
    """One mi_decode_step_static call with the decoder's model parameters."""
    import torch
    from mamba_int import _lib
    n = dec.params.n_layer
    conv = (ctypes.c_void_p * n)(*[c.data_ptr() for c in state.conv])
    h = (ctypes.c_void_p * n)(*[t.data_ptr() for t in state.h])
    _lib.call("mi_decode_step_static", dec._pp, dec.m, ctypes.c_void_p(ids.data_ptr()),
              ctypes.c_void_p(next_ids.data_ptr()), ctypes.c_void_p(logits.data_ptr()), logits.stride(0),
              ctypes.cast(conv, ctypes.c_void_p), ctypes.cast(h, ctypes.c_void_p),
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.gpu
@pytest.mark.parametrize("d_model,n_layer,vocab", [(768, 3, 32000), (2048, 2, 32000)])
def test_static_step_matches_workspace_step(cuda, d_model, n_layer, vocab):
    """Two runs in a row (batch 8, then the smaller batch 3) of four chained
    greedy steps each: ids, logits and the recurrent state agree with
    mi_decode_step's after every step.  d768 runs the fused stages, d2048 the
    batched ones (the two layouts of the workspace)."""
    import torch
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    run = IntegerMambaRunner(_model(d_model, n_layer, vocab))
    rng = np.random.default_rng(d_model)
    for m in (8, 3):
        ids = torch.from_numpy(rng.integers(0, vocab, size=(m, 12))).cuda()
        logits0, st_a = run.prefill(ids)
        st_b = st_a.clone()
        dec = NativeDecoder(run, m)
        tok_a = ops.argmax(logits0)
        tok_b = tok_a.clone()
        for _ in range(4):
            nxt_a = torch.empty_like(tok_a)
            nxt_b = torch.full_like(tok_b, -1)
            lg_a = torch.empty((m, vocab), dtype=torch.int32, device="cuda")
            lg_b = torch.full((m, vocab), -7, dtype=torch.int32, device="cuda")
            dec.step(tok_a, st_a, nxt_a, lg_a)
            _static_step(dec, tok_b, st_b, nxt_b, lg_b)
            torch.cuda.synchronize()
            assert torch.equal(nxt_a, nxt_b)
            assert torch.equal(lg_a, lg_b)
            for i in range(n_layer):
                assert torch.equal(st_a.conv[i], st_b.conv[i]) and torch.equal(st_a.h[i], st_b.h[i])
            tok_a, tok_b = nxt_a, nxt_b


def _static_raw(dec, ids, state, next_ids, logits, stream):
    """mi_decode_step_static on `stream`, returning its status instead of raising."""
    from mamba_int import _lib
    n = dec.params.n_layer
    conv = (ctypes.c_void_p * n)(*[c.data_ptr() for c in state.conv])
    h = (ctypes.c_void_p * n)(*[t.data_ptr() for t in state.h])
    return _lib.raw("mi_decode_step_static", dec._pp, dec.m, ctypes.c_void_p(ids.data_ptr()),
                    ctypes.c_void_p(next_ids.data_ptr()), ctypes.c_void_p(logits.data_ptr()), logits.stride(0),
                    ctypes.cast(conv, ctypes.c_void_p), ctypes.cast(h, ctypes.c_void_p),
                    ctypes.c_void_p(stream.cuda_stream))


@pytest.mark.gpu
def test_static_step_captured_in_a_graph(cuda):
    """One eager call sets the device up; two static steps captured in a
    torch.cuda graph then replay three times, with eager work and
    synchronizations between the replays, and after every replay the ids, the
    logits and the recurrent state equal two mi_decode_step steps."""
    import torch
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    m, V, nl = 8, 32000, 3
    run = IntegerMambaRunner(_model(768, nl, V))
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, V, size=(m, 10))).cuda()
    logits0, st_a = run.prefill(ids)
    dec = NativeDecoder(run, m)
    tok_a = ops.argmax(logits0)
    st_b, tok_b = st_a.clone(), tok_a.clone()
    nxt_b = torch.empty_like(tok_b)
    lg_b = torch.empty((m, V), dtype=torch.int32, device="cuda")
    warm = st_a.clone()                                  # set-up call, outside capture
    _static_step(dec, tok_a.clone(), warm, torch.empty_like(tok_a), torch.empty_like(lg_b))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _static_step(dec, tok_b, st_b, nxt_b, lg_b)
        _static_step(dec, nxt_b, st_b, tok_b, lg_b)
    for _ in range(3):
        g.replay()
        for _ in range(2):                              # the reference: two workspace steps, eager
            nxt_a = torch.empty_like(tok_a)
            lg_a = torch.empty((m, V), dtype=torch.int32, device="cuda")
            dec.step(tok_a, st_a, nxt_a, lg_a)
            tok_a = nxt_a
        torch.cuda.synchronize()
        assert torch.equal(tok_b, tok_a) and torch.equal(lg_b, lg_a)
        for i in range(nl):
            assert torch.equal(st_a.conv[i], st_b.conv[i]) and torch.equal(st_a.h[i], st_b.h[i])


@pytest.mark.gpu
def test_static_step_refuses_an_overlapping_call(cuda):
    """A call on stream B while the previous call, on stream A, is still queued
    (behind a bounded spin kernel) is refused with MI_ERR_BAD_ARG and enqueues
    nothing; once A has finished, the call on B runs and equals the workspace step."""
    import torch
    from mamba_int import _lib, ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeDecoder
    m, V = 4, 4000
    run = IntegerMambaRunner(_model(256, 2, V))
    ids = torch.from_numpy(np.random.default_rng(4).integers(0, V, size=(m, 6))).cuda()
    logits0, st = run.prefill(ids)
    dec = NativeDecoder(run, m)
    tok = ops.argmax(logits0)
    st_ref, st_a, st_b = st.clone(), st.clone(), st.clone()
    lg = torch.empty((m, V), dtype=torch.int32, device="cuda")
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    nxt_a = torch.empty_like(tok)
    with torch.cuda.stream(sa):
        torch.cuda._sleep(200_000_000)                  # a bounded spin ahead of the call on A
    assert _static_raw(dec, tok, st_a, nxt_a, lg, sa) == 0
    nxt_b = torch.full_like(tok, -1)
    assert _static_raw(dec, tok, st_b, nxt_b, lg, sb) == 4
    assert "still running" in _lib.last_error()
    sa.synchronize()
    sb.synchronize()
    assert (nxt_b == -1).all()                          # the refused call enqueued nothing
    assert _static_raw(dec, tok, st_b, nxt_b, lg, sb) == 0
    sb.synchronize()
    nxt_ref = torch.empty_like(tok)
    dec.step(tok, st_ref, nxt_ref)
    torch.cuda.synchronize()
    assert torch.equal(nxt_a, nxt_ref) and torch.equal(nxt_b, nxt_ref)
    for i in range(2):
        assert torch.equal(st_b.h[i], st_ref.h[i]) and torch.equal(st_a.h[i], st_ref.h[i])


def test_static_step_rejects_a_workspace_beyond_the_scratch():
    """A model whose workspace exceeds the 16 MiB static array is refused before
    anything reaches a device (runs without a GPU)."""
    from mamba_int import _lib
    from mamba_int.native import ModelParams
    p = ModelParams(3072, 2, 1 << 20, 16, 64, 0x1000, None, 0x1000, 0x1000)
    p.layers = ctypes.cast(ctypes.c_void_p(0x1000), type(p.layers))
    pp = ctypes.cast(ctypes.pointer(p), ctypes.c_void_p)
    n = ctypes.c_size_t(0)
    assert _lib.raw("mi_decode_workspace_size", pp, 64, ctypes.cast(ctypes.pointer(n), ctypes.c_void_p)) == 0
    assert n.value > 16 << 20
    A = ctypes.c_void_p(0x1000)
    st = _lib.raw("mi_decode_step_static", pp, 64, A, A, None, 0, A, A, None)
    assert st == 2 and "static scratch holds 16777216" in _lib.last_error()
    # the d768 x 24 and d2048 x 48 models of the benchmarks fit at batch 64
    for d, nl, dr in ((768, 24, 48), (2048, 48, 128)):
        q = ModelParams(d, nl, 32000, 16, dr, 0x1000, None, 0x1000, 0x1000)
        q.layers = p.layers
        qq = ctypes.cast(ctypes.pointer(q), ctypes.c_void_p)
        assert _lib.raw("mi_decode_workspace_size", qq, 64, ctypes.cast(ctypes.pointer(n), ctypes.c_void_p)) == 0
        assert n.value <= 16 << 20, (d, n.value)
