"""The reference's model-loading flow on the drop-in modules.

scripts/inference.py:103-121 builds ``MambaIntegerModel(config)``, unwraps a
nested ``model_state_dict``, strips the ``_orig_mod.`` prefix and calls
``model.load_state_dict(new_state_dict, strict=False)``.  On the drop-in that
call converts the float state dict to the integer parameters (the converter's
rules are pinned in test_checkpoint.py) and installs them; a state dict it
cannot convert raises instead of leaving random weights in place.  The GPU
tests check that the loaded model computes what ``from_checkpoint`` on the
converted file computes, and the float faces of the block and the norm.
"""
import numpy as np
import pytest
import torch

import oracle as O
from mamba_int import checkpoint as ckpt
from mamba_int.params import ModelParams
from test_checkpoint import DIMS, SSD_DIMS, _config, _ssd_config, _ssd_state_dict, _state_dict


def _equal_params(p, q):
    assert p.dims == q.dims
    for k in ("emb", "gamma_f", "w_head"):
        assert np.array_equal(getattr(p, k), getattr(q, k)), k
    for a, b in zip(p.layers, q.layers):
        for k in a.__dataclass_fields__:
            assert np.array_equal(getattr(a, k), getattr(b, k)), k


def _reference_flow(model, checkpoint):
    """The loading steps of scripts/inference.py:107-121, verbatim in effect."""
    state_dict = checkpoint["model_state_dict"] if "model_state_dict" in checkpoint else checkpoint
    new_state_dict = {}
    for k, v in state_dict.items():
        new_state_dict[k[10:] if k.startswith("_orig_mod.") else k] = v
    return model.load_state_dict(new_state_dict, strict=False)


@pytest.mark.parametrize("ssd", [False, True])
def test_reference_loader_flow_installs_the_weights(ssd):
    from mamba_integer_model import MambaIntegerModel
    sd = _ssd_state_dict(np.random.default_rng(4)) if ssd else _state_dict(np.random.default_rng(3))
    cfg = _ssd_config() if ssd else _config()
    want, want_scale = ckpt.convert_state_dict(sd, cfg)
    model = MambaIntegerModel(cfg)
    res = _reference_flow(model, {"model_state_dict": {"_orig_mod." + k: v for k, v in sd.items()}})
    assert res.missing_keys == [] and res.unexpected_keys == []
    _equal_params(model.params, want)
    assert model.logit_scale == want_scale and model.dims == want.dims


def test_load_state_dict_strictness():
    """Unused keys: returned under strict=False, refused under strict=True.  A
    missing tensor, a wrong shape or an unrepresentable value raises either way
    and leaves the model's parameters as they were."""
    from mamba_integer_model import MambaIntegerModel
    sd = _state_dict(np.random.default_rng(5))
    sd["layers.0.mystery"] = torch.zeros(3)
    model = MambaIntegerModel(_config(), seed=1)
    res = model.load_state_dict(sd, strict=False)
    assert res.unexpected_keys == ["layers.0.mystery"]
    with pytest.raises(RuntimeError, match="Unexpected key"):
        MambaIntegerModel(_config()).load_state_dict(sd, strict=True)
    before = MambaIntegerModel(_config(), seed=1)
    p0 = before.params
    for change in ("drop", "shape", "shifts"):
        bad = _state_dict(np.random.default_rng(5))
        if change == "drop":
            del bad["layers.1.out_proj.weight"]
        elif change == "shape":
            bad["embedding.weight"] = bad["embedding.weight"][:, :32]
        else:
            bad["layers.0.decay_shifts"][0, 0] = 14.0
        with pytest.raises(ckpt.CheckpointError):
            before.load_state_dict(bad, strict=False)
        assert before.params is p0


def test_block_and_norm_load_state_dict():
    """MambaIntegerBlock / MambaIntegerBlockV2 take one block's float state dict
    (no layers.{i}. prefix); BitShiftNorm takes gamma and step_size."""
    from mamba_integer_model import BitShiftNorm, MambaIntegerBlock, MambaIntegerBlockV2
    for ssd in (False, True):
        sd = _ssd_state_dict(np.random.default_rng(6)) if ssd else _state_dict(np.random.default_rng(6))
        cfg = _ssd_config() if ssd else _config()
        full, _ = ckpt.convert_state_dict(sd, cfg)
        blk_sd = {k[len("layers.1."):]: v for k, v in sd.items() if k.startswith("layers.1.")}
        blk = (MambaIntegerBlockV2 if ssd else MambaIntegerBlock)(cfg, 1)
        assert blk.load_state_dict(blk_sd).unexpected_keys == []
        for k in full.layers[1].__dataclass_fields__:
            assert np.array_equal(getattr(blk.params, k), getattr(full.layers[1], k)), (ssd, k)
        with pytest.raises(RuntimeError):
            blk.load_state_dict(dict(blk_sd, extra=torch.zeros(1)), strict=True)
    norm = BitShiftNorm(DIMS.d_model)
    g = torch.from_numpy(np.random.default_rng(7).uniform(0.5, 1.5, DIMS.d_model).astype(np.float32))
    norm.load_state_dict({"gamma": g, "step_size": torch.tensor([0.75])})
    assert torch.equal(norm.gamma_q, torch.round(g * np.float32(0.75) * 256).to(torch.int16))


# ------------------------------------------------------------------ GPU
def _T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("ssd", [False, True])
def test_gpu_loaded_model_equals_from_checkpoint(cuda, tmp_path, ssd):
    """After the reference's load flow the drop-in's logits and greedy tokens equal
    those of from_checkpoint on the converted file (and the oracle's)."""
    from mamba_integer_model import MambaIntegerModel
    if ssd:
        sd, cfg, V = _ssd_state_dict(np.random.default_rng(8)), _ssd_config(), SSD_DIMS.vocab_size
    else:
        sd, cfg, V = _state_dict(np.random.default_rng(8)), _config(), DIMS.vocab_size
    torch.save(sd, tmp_path / "ref.pt")
    ckpt.convert_reference_checkpoint(str(tmp_path / "ref.pt"), cfg, str(tmp_path / "c.miq"))
    ref_model = MambaIntegerModel.from_checkpoint(str(tmp_path / "c.miq"))
    model = MambaIntegerModel(cfg).to("cuda")
    _reference_flow(model, torch.load(tmp_path / "ref.pt", weights_only=True))
    ids = _T(np.random.default_rng(9).integers(0, V, size=(2, 14)))
    got = model(ids)
    assert torch.equal(got, ref_model(ids))
    want = O.OracleModel(ref_model.params).forward(ids.cpu().numpy())
    assert np.array_equal(model.forward_int(ids).cpu().numpy(), want)
    assert torch.equal(model.generate(ids, 5), ref_model.generate(ids, 5))


@pytest.mark.gpu
@pytest.mark.parametrize("ssd", [False, True])
def test_gpu_block_and_norm_float_faces(cuda, ssd):
    """MambaIntegerBlock.forward on float hidden states = the integer block on
    round_half_even(x * 256) (saturated to the Q8 range), returned / 256, and
    equal to the oracle's layer; BitShiftNorm's float face = the integer norm of
    the same Q8 input / 16."""
    from mamba_integer_model import (BitShiftNorm, BitShiftNormV2, MambaIntegerBlock, MambaIntegerBlockV2,
                                     to_q8)
    cfg = _ssd_config() if ssd else _config()
    dims = SSD_DIMS if ssd else DIMS
    blk = (MambaIntegerBlockV2 if ssd else MambaIntegerBlock)(cfg, 0, seed=3)
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((2, 11, dims.d_model)) * rng.choice([0.01, 1.0, 30.0, 5e4], (2, 11, 1)))
    x = x.astype(np.float32)
    x[0, 0, :4] = [0.5 / 256, 1.5 / 256, -2.5 / 256, 1e9]          # ties to even, and saturation
    q = to_q8(torch.from_numpy(x))
    assert q[0, 0, :4].tolist() == [0, 2, -2, 2**23 - 1]
    out = blk(_T(x))
    assert out.dtype == torch.float32
    want_int = blk.forward_int(_T(q.numpy()))
    assert torch.equal(out, want_int.to(torch.float32) / 256)
    r = q.numpy().reshape(-1, dims.d_model)
    om = O.OracleModel(ModelParams(dims=dims, emb=None, layers=[blk.params]))
    ref, _ = om._layer(blk.params, r, 2, 11, None)
    assert np.array_equal(want_int.cpu().numpy().reshape(-1, dims.d_model), ref)
    norm = (BitShiftNormV2 if ssd else BitShiftNorm)(dims.d_model)
    y = norm(_T(x))
    want = (O.bitshift_norm_v2 if ssd else O.bitshift_norm)(r, norm.gamma_q.numpy()).astype(np.float32) / 16
    assert np.array_equal(y.cpu().numpy().reshape(-1, dims.d_model), want)
