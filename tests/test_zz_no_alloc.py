"""mi_decode_step_static: the whole greedy decode step with the library's
static device workspace (no allocation), against mi_decode_step with a
caller-owned workspace, bit for bit, through the C ABI."""
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
