"""The prefill in_proj with the conv + squareplus of its x half fused into the
GEMM epilogue (mi_in_proj_conv) against the oracle's BitLinear (int8 requant)
followed by its conv + squareplus, bit for bit: xs, the z half and the conv
state.  The x-half tiles store 125 of their 128 rows (the first three are the
conv window of the tile's first row), so the cases put sequence starts and
ends on both sides of tile edges, and sequences shorter than the window."""
import numpy as np
import pytest

import oracle as O
from conftest import i8

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("B,L,d,D,with_state", [
    (1, 1, 64, 128, False),
    (3, 1, 64, 128, True),
    (2, 2, 128, 128, True),      # sequences shorter than the conv window
    (4, 3, 64, 256, True),
    (2, 125, 64, 128, False),    # one x tile per sequence
    (1, 126, 64, 128, True),     # one row past the first tile
    (3, 130, 192, 256, True),    # sequences straddle tiles; K tail (192 = 128 + 64)
    (5, 77, 768, 128, True),
    (2, 400, 64, 384, False),
    (1, 1000, 128, 128, True),
    # d_inner % 256 == 0, d_model % 128 == 0 and at least 512 tiles: the 256 x 128-tile form
    (4, 4100, 128, 512, True),   # sequences straddle x tiles of 125 rows
    (1, 16400, 256, 512, False),
    (8200, 2, 128, 512, True),   # sequences shorter than the conv window
    (2, 8193, 768, 512, True),
])
def test_in_proj_conv_matches_oracle(cuda, B, L, d, D, with_state):
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(B * 1000 + L + d + D)
    M = B * L
    a = i8(rng, M, d)
    wp = O.pack_ternary(rng.integers(-1, 2, size=(2 * D, d), dtype=np.int8))
    shift = 5
    cw = i8(rng, D, 4)
    cb = rng.integers(-60000, 60000, size=D, dtype=np.int32)   # reaches the +-51200 clamp
    st = i8(rng, B, 3, D) if with_state else None
    xz_ref = O.bitlinear(a, wp, O.OUT_INT8, shift)
    xs_ref, st_ref = O.conv_squareplus(xz_ref.reshape(B, L, 2 * D), D, cw, cb, st)

    st_out = torch.full((B, 3, D), 0x55, dtype=torch.int8, device="cuda")
    xz = torch.full((M, 2 * D), 0x33, dtype=torch.int8, device="cuda")
    xs, xz = ops.in_proj_conv(T(a), T(wp), shift, D, T(cw), T(cb), B, st_out,
                              state_in=None if st is None else T(st), xz=xz)
    assert np.array_equal(H(xs), xs_ref.reshape(M, D))
    assert np.array_equal(H(xz)[:, D:], xz_ref[:, D:])
    assert (H(xz)[:, :D] == 0x33).all()          # the x half is not written
    assert np.array_equal(H(st_out), st_ref)


def test_in_proj_conv_rejects_overlapping_states(cuda):
    import torch
    from mamba_int import _lib, ops
    B, L, d, D = 2, 8, 64, 128
    st = torch.zeros((B, 3, D), dtype=torch.int8, device="cuda")
    a = torch.zeros((B * L, d), dtype=torch.int8, device="cuda")
    wp = torch.zeros((2 * D, d // 4), dtype=torch.uint8, device="cuda")
    cw = torch.zeros((D, 4), dtype=torch.int8, device="cuda")
    cb = torch.zeros((D,), dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.MIError, match="overlap"):
        ops.in_proj_conv(a, wp, 5, D, cw, cb, B, st, state_in=st)


@pytest.mark.parametrize("with_state", [True, False])
def test_in_proj_conv_no_rows_carries_state(cuda, with_state):
    """len = 0: no row is computed and state_out receives state_in unchanged (zeros
    when state_in is None), as a sequence with no new rows keeps its conv window."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(11)
    B, d, D = 3, 64, 256
    wp = O.pack_ternary(rng.integers(-1, 2, size=(2 * D, d), dtype=np.int8))
    cw, cb = i8(rng, D, 4), rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, B, 3, D)
    st_out = torch.full((B, 3, D), 0x55, dtype=torch.int8, device="cuda")
    a = torch.empty((0, d), dtype=torch.int8, device="cuda")
    xs, xz = ops.in_proj_conv(a, T(wp), 5, D, T(cw), T(cb), B, st_out,
                              state_in=T(st) if with_state else None)
    assert xs.shape == (0, D) and xz.shape == (0, 2 * D)
    assert np.array_equal(H(st_out), st if with_state else np.zeros_like(st))
