"""Integer checkpoints on the GPU: the native loader's upload drives the
whole decode step (mi_decode_step) to the oracle's greedy continuation, and a
model converted from a float state dict runs bit-exact against the oracle on
the converted integers."""
import numpy as np
import pytest

import oracle as O
from mamba_int import ModelDims, checkpoint as ckpt, init_random_params

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


def test_native_checkpoint_upload_decodes(cuda, tmp_path):
    """mi_checkpoint_open + mi_checkpoint_upload -> mi_decode_step: the device
    buffer holds the file's tensors at the 256-byte layout, and greedy decode
    from it equals the oracle on the same parameters."""
    import torch
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeCheckpoint
    p = init_random_params(ModelDims(d_model=128, n_layer=3, vocab_size=500, d_state=16, dt_rank=16), 31)
    path = tmp_path / "m.miq"
    ckpt.save(p, str(path), 0.01)
    ck = NativeCheckpoint(str(path), device="cuda")
    buf = H(ck.buffer)
    assert np.array_equal(buf[:p.emb.nbytes].view(np.int8).reshape(p.emb.shape), p.emb)
    off = -(-p.emb.nbytes // 256) * 256
    assert np.array_equal(buf[off:off + p.gamma_f.nbytes].view(np.int16), p.gamma_f)
    assert ck.params.layers[2].s_in == p.layers[2].s_in and ck.params.layers[1].res_mult == p.layers[1].res_mult
    ids = np.random.default_rng(5).integers(0, 500, size=(2, 9))
    ref = O.OracleModel(p).generate(ids, 8)
    run = IntegerMambaRunner(p)
    lg, st = run.prefill(T(ids))
    dec = ck.decoder(2)
    assert np.array_equal(H(dec.generate(ops.argmax(lg), st, 8)), ref)
    torch.cuda.synchronize()


def test_converted_float_checkpoint_matches_oracle(cuda, tmp_path):
    """A float state dict in the reference's key layout, converted and written
    as a format-1 file, loads into the runner and the drop-in model; prefill
    logits and greedy decode equal the oracle on the converted integers."""
    import torch
    from test_checkpoint import _config, _state_dict
    from mamba_integer_model import MambaIntegerModel
    dims = ModelDims(d_model=128, n_layer=2, vocab_size=300, d_state=16, dt_rank=16)
    sd = _state_dict(np.random.default_rng(7), dims)
    torch.save(sd, tmp_path / "ref.pt")
    ckpt.convert_reference_checkpoint(str(tmp_path / "ref.pt"), _config(dims), str(tmp_path / "c.miq"))
    model = MambaIntegerModel.from_checkpoint(str(tmp_path / "c.miq"))
    p = model.params
    ids = np.random.default_rng(9).integers(0, 300, size=(2, 16))
    om = O.OracleModel(p)
    ref_logits = om.forward(ids)
    got = model.forward_int(T(ids))
    assert np.array_equal(H(got), ref_logits)
    flt = model(T(ids))
    assert torch.equal(flt, got.to(torch.float32) * model.logit_scale)
    assert np.array_equal(H(model.generate(T(ids), 6))[:, 16:], om.generate(ids, 6))


def test_ssd_checkpoint_native_decode_and_conversion(cuda, tmp_path):
    """The multi-head SSD block through the file format: a random model decodes
    natively (mi_checkpoint_upload -> mi_decode_step, the per-op SSD path) to
    the oracle's greedy continuation, the runner-built native decoder agrees,
    and a converted V2 float state dict matches the oracle's logits."""
    import torch
    from test_checkpoint import _ssd_config, _ssd_state_dict
    from mamba_int import ops
    from mamba_int.model import IntegerMambaRunner
    from mamba_int.native import NativeCheckpoint, NativeDecoder
    from mamba_integer_model import MambaIntegerModel
    dims = ModelDims(d_model=128, n_layer=2, vocab_size=500, d_state=32, dt_rank=0, block="ssd", n_heads=4,
                     d_head=64)
    p = init_random_params(dims, 17)
    path = tmp_path / "v2.miq"
    ckpt.save(p, str(path), 0.01)
    ids = np.random.default_rng(6).integers(0, 500, size=(3, 10))
    ref = O.OracleModel(p).generate(ids, 8)
    run = IntegerMambaRunner(p)
    lg, st = run.prefill(T(ids))
    first = ops.argmax(lg)
    ck = NativeCheckpoint(str(path), device="cuda")
    assert ck.params.block == 1 and ck.params.layers[1].decay_tab
    assert np.array_equal(H(ck.decoder(3).generate(first, st.clone(), 8)), ref)
    assert np.array_equal(H(NativeDecoder(run, 3).generate(first, st, 8)), ref)
    sd = _ssd_state_dict(np.random.default_rng(8))
    torch.save(sd, tmp_path / "v2.pt")
    ckpt.convert_reference_checkpoint(str(tmp_path / "v2.pt"), _ssd_config(), str(tmp_path / "c2.miq"))
    model = MambaIntegerModel.from_checkpoint(str(tmp_path / "c2.miq"))
    ids = np.random.default_rng(9).integers(0, 90, size=(2, 12))
    assert np.array_equal(H(model.forward_int(T(ids))), O.OracleModel(model.params).forward(ids))
