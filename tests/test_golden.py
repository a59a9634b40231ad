"""Golden fixtures (tests/golden/*.npz, written by make_golden.py from an
independent pure-Python restatement) against the CPU oracle and the GPU path."""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name)) as f:
        return {k: f[k] for k in f.files}


def test_oracle_scan():
    g = load("scan_c1_small.npz")
    y, h = O.dyadic_scan(g["x"], g["b"], g["c"], g["n"], 15, h_state=g["h0"])
    assert np.array_equal(y, g["y"]) and np.array_equal(h, g["h"])


def test_oracle_ssd():
    g = load("ssd_small.npz")
    assert np.array_equal(O.ssd_chunked_scan(g["x"], g["b"], g["c"], g["n"], 15, int(g["chunk"])), g["y"])


def test_oracle_bitlinear_and_packing():
    g = load("bitlinear_small.npz")
    assert np.array_equal(O.pack_ternary(g["w"]), g["packed"])
    assert np.array_equal(O.bitlinear(g["a"], g["packed"], O.OUT_INT32), g["acc"])
    assert np.array_equal(O.bitlinear(g["a"], g["packed"], O.OUT_INT8, 5), g["q5"])


def test_oracle_norm():
    g = load("norm_small.npz")
    assert np.array_equal(O.bitshift_norm(g["r"], g["gamma"]), g["out"])


def test_oracle_conv_sqp():
    g = load("conv_sqp_small.npz")
    xs, st = O.conv_squareplus(g["x"], 16, g["w"], g["bias"], g["state"])
    assert np.array_equal(xs, g["xs"]) and np.array_equal(st, g["state_out"])


def test_oracle_block_scan():
    g = load("block_scan_small.npz")
    yo, h = O.block_scan(g["xs"], g["dm"], g["xp"], 16, g["z"], 0, g["base"], 15, 13, h_state=g["h0"])
    assert np.array_equal(yo, g["yo"]) and np.array_equal(h, g["h"])


@pytest.mark.gpu
def test_gpu_matches_golden(cuda):
    import torch
    from mamba_int import ops

    def T(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    g = load("scan_c1_small.npz")
    h = T(g["h0"])
    y = ops.dyadic_scan(T(g["x"]), T(g["b"]), T(g["c"]), T(g["n"]), 15, h_in=h, h_out=h)
    assert np.array_equal(y.cpu().numpy(), g["y"]) and np.array_equal(h.cpu().numpy(), g["h"])
    g = load("ssd_small.npz")
    y = ops.ssd_chunked_scan(T(g["x"]), T(g["b"]), T(g["c"]), T(g["n"]), 15, int(g["chunk"]))
    assert np.array_equal(y.cpu().numpy(), g["y"])
    g = load("bitlinear_small.npz")
    assert np.array_equal(ops.pack_ternary(T(g["w"])).cpu().numpy(), g["packed"])
    for path in ("gemm", "gemv"):
        acc = ops.bitlinear(T(g["a"]), T(g["packed"]), ops.OUT_INT32, 20, path=path)
        assert np.array_equal(acc.cpu().numpy(), g["acc"])
    g = load("norm_small.npz")
    assert np.array_equal(ops.bitshift_norm(T(g["r"]), T(g["gamma"])).cpu().numpy(), g["out"])
    g = load("conv_sqp_small.npz")
    st = T(g["state"])
    xs = ops.conv_squareplus(T(g["x"]), 16, T(g["w"]), T(g["bias"]), state_in=st, state_out=st)
    assert np.array_equal(xs.cpu().numpy(), g["xs"]) and np.array_equal(st.cpu().numpy(), g["state_out"])
    g = load("block_scan_small.npz")
    h = T(g["h0"])
    yo = ops.block_scan(T(g["xs"]), T(g["dm"]), T(g["xp"]), 16, T(g["z"]), 0, T(g["base"]), 15, 13, h_in=h, h_out=h)
    assert np.array_equal(yo.cpu().numpy(), g["yo"]) and np.array_equal(h.cpu().numpy(), g["h"])
