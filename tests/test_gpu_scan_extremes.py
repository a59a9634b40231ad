"""GPU parity of the fast scan kernels at the edges of their state arithmetic.

The fast kernels read the int32 state as two 16-bit fields (H = h >> 16,
L = h & 0xffff) and the decay as n2 = 2n, so the products meet their bounds at
H = -2^15 or 2^15 - 1, L = 0xffff and n = 2^15 (n2 = 2^16).  These tests start
from states spread over the whole int32 range (INT32_MIN and INT32_MAX
included), take decays 0, 1, 2^15 - 1 and 2^15 (or the model's clamp edges),
drive chosen lanes into both saturation directions, and compare every output
and the final state with the oracle, bit for bit."""
import numpy as np
import pytest

import oracle as O
from conftest import i8

pytestmark = pytest.mark.gpu

I32_MIN, I32_MAX = -2**31, 2**31 - 1


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


def _full_range_states(rng, shape):
    h = rng.integers(I32_MIN, I32_MAX + 1, size=shape, dtype=np.int64).astype(np.int32)
    flat = h.reshape(-1)
    flat[0::7] = I32_MAX
    flat[1::7] = I32_MIN
    flat[2::11] = I32_MAX - 1
    flat[3::11] = I32_MIN + 1
    flat[4::13] = -1
    flat[5::13] = 0x7fff0000
    flat[6::13] = -0x8000 * 0x10000 + 0xffff
    return h


@pytest.mark.parametrize("N", [16, 32, 64, 128])
def test_channel_scan_state_extremes(cuda, N):
    """mi_dyadic_scan (fast path: k = 15, d % 16 == 0) from full-range states;
    channel 0 saturates up, channel 1 down, at decay 2^15."""
    from mamba_int import ops
    rng = np.random.default_rng(100 + N)
    B, L, D = 2, 150, 32
    x = i8(rng, B, L, D, lo=-128)
    b = i8(rng, B, L, N, lo=-128)
    c = i8(rng, B, L, N, lo=-128)
    n = rng.choice(np.array([0, 1, 2, 16384, 32767, 32768], np.int32), size=(D, N))
    n[:, ::3] = rng.integers(0, 32769, size=(D, n[:, ::3].shape[1]), dtype=np.int32)
    h0 = _full_range_states(rng, (B, D, N))
    x[:, :, 0], x[:, :, 1] = 127, -128
    b[:, :, 0] = 127
    n[0, 0] = n[1, 0] = 32768
    h0[:, 0, 0], h0[:, 1, 0] = I32_MAX - 5, I32_MIN + 5
    y_ref, h_ref = O.dyadic_scan(x, b, c, n, 15, h_state=h0)
    assert (h_ref[:, 0, 0] == I32_MAX).all() and (h_ref[:, 1, 0] == I32_MIN).all()
    hout = T(np.zeros_like(h0))
    y = ops.dyadic_scan(T(x), T(b), T(c), T(n), 15, h_in=T(h0), h_out=hout)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(hout), h_ref)


def test_ssd_chunked_scan_state_extremes(cuda):
    """mi_ssd_chunked_scan at the config-4 layout (N 128, head_dim 64, the fast
    path) from full-range states, one head at each decay edge: y, every chunk
    state and the final state."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(41)
    B, L, H_, P, N, cs = 2, 300, 4, 64, 128, 128
    x = i8(rng, B, L, H_, P, lo=-128)
    b = i8(rng, B, L, H_, N, lo=-128)
    c = i8(rng, B, L, H_, N, lo=-128)
    n = np.array([32768, 0, 1, 32767], np.int32)
    h0 = _full_range_states(rng, (B, H_, P, N))
    x[:, :, 0, 0], x[:, :, 0, 1] = 127, -128
    b[:, :, 0, 0] = 127
    h0[:, 0, 0, 0], h0[:, 0, 1, 0] = I32_MAX - 5, I32_MIN + 5
    y_ref, cs_ref, h_ref = O.ssd_chunked_scan(x, b, c, n, 15, cs, want_chunk_states=True, h_state=h0)
    assert h_ref[:, 0, 0, 0].tolist() == [I32_MAX] * B and h_ref[:, 0, 1, 0].tolist() == [I32_MIN] * B
    nc = -(-L // cs)
    cst = torch.empty((B, nc, H_, P, N), dtype=torch.int32, device="cuda")
    hout = torch.empty((B, H_, P, N), dtype=torch.int32, device="cuda")
    y = ops.ssd_chunked_scan(T(x), T(b), T(c), T(n), 15, cs, chunk_states=cst, h_in=T(h0), h_out=hout)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(cst), cs_ref)
    assert np.array_equal(H(hout), h_ref)


@pytest.mark.parametrize("N,B,L,D", [(16, 2, 140, 256), (32, 2, 140, 256), (16, 32, 70, 1536), (16, 8, 70, 1536),
                                     (16, 6, 50, 1504)])
def test_block_scan_state_extremes(cuda, N, B, L, D):
    """mi_block_scan (the fused prefill scan) from full-range states, bases at
    the clamp edges 0 and 32000 (and within 20 of them, so some waves take the
    clamped decay and some the unclamped one), dm over its whole range.  The
    32 x 1536 case takes the 4-lanes-per-channel layout (batch x d_inner >=
    49152); 8 x 1536 and 6 x 1504 the mixed 48-channel block (8 lanes a
    channel in one half, 16 in the other; 1504 ends in a block with 16 of its
    48 channels); the others 8 lanes."""
    from mamba_int import ops
    rng = np.random.default_rng(200 + N + B)
    R = 16
    W = (R + 2 * N + 15) // 16 * 16
    xs = i8(rng, B, L, D, lo=-128)
    dm = i8(rng, B, L, D, lo=-128)
    xp = i8(rng, B, L, W, lo=-128)
    z = i8(rng, B, L, 2 * D, lo=-128)
    base = rng.integers(20, 31981, size=(D, N), dtype=np.int32)   # channels 0..127: every wave clamp-free
    base[128:] = rng.choice(np.array([0, 1, 19, 31981, 31999, 32000], np.int32), size=(D - 128, N))
    h0 = _full_range_states(rng, (B, D, N))
    yo_ref, h_ref = O.block_scan(xs, dm, xp, R, z, D, base, 15, 14, h_state=h0)
    hg = T(h0)
    yo = ops.block_scan(T(xs), T(dm), T(xp), R, T(z), D, T(base), 15, 14, h_in=hg, h_out=hg)
    assert np.array_equal(H(yo), yo_ref)
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("L", [1, 90])
def test_ssd_block_scan_state_extremes(cuda, L):
    """mi_ssd_block_scan from full-range states with decay-table entries 0 and
    2^15 among random ones, and one head driven into both saturation directions
    (the clamped multiply-add of the input term): the chunked kernel (L 90) and
    the one-step kernel (L 1)."""
    from mamba_int import ops
    rng = np.random.default_rng(300 + L)
    B, Hh, P, N = 2, 3, 32, 64
    D = Hh * P
    W = -(-(2 * Hh * N + Hh) // 16) * 16
    xs = i8(rng, B, L, D, lo=-128)
    xp = i8(rng, B, L, W, lo=-128)
    xz = i8(rng, B, L, 2 * D, lo=-128)
    tab = rng.integers(0, 32769, size=(Hh, 255)).astype(np.int32)
    tab[:, ::4] = 32768
    tab[:, 1::4] = 0
    h0 = _full_range_states(rng, (B, D, N))
    # head 0 keeps its state (decay 2^15 at every dt) and takes a positive unit
    # B: channel 0 (x = 127) saturates up, channel 1 (x = -128) down
    tab[0] = 32768
    xp[:, :, :N] = 127
    xs[:, :, 0], xs[:, :, 1] = 127, -128
    h0[:, 0], h0[:, 1] = I32_MAX - 5, I32_MIN + 5
    ref_y, ref_h = O.ssd_v2_scan(xs, xp, xz, D, tab, 14, Hh, N, h_state=h0)
    assert (ref_h[:, 0] == I32_MAX).all() and (ref_h[:, 1] == I32_MIN).all()
    h = T(h0)
    y = ops.ssd_block_scan(T(xs), T(xp), T(xz), D, T(tab), Hh, N, 14, h_in=h, h_out=h)
    assert np.array_equal(H(y), ref_y)
    assert np.array_equal(H(h), ref_h)


@pytest.mark.parametrize("B,L,D", [(8, 77, 1520), (8, 77, 1552), (1, 33, 8208), (3, 5, 3072)])
def test_block_scan_mixed_route_edges(cuda, B, L, D):
    """mi_block_scan from a zero state (no h_in) at the edges of the mixed
    48-channel block's route (batch x d_inner > 8192 and batch x
    ceil(d_inner / 48) <= 256): 8 x 1520 ends in a block whose 16-lane half
    has no channel, 8 x 1552 needs 264 blocks and keeps 8 lanes a channel,
    1 x 8208 runs 171 mixed blocks, 3 x 3072 192 of them; L not a multiple
    of 4 or 64."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(B * L + D)
    N, R = 16, 48
    W = R + 2 * N
    xs = i8(rng, B, L, D, lo=-128)
    dm = i8(rng, B, L, D, lo=-128)
    xp = i8(rng, B, L, W, lo=-128)
    z = i8(rng, B, L, 2 * D, lo=-128)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    yo_ref, h_ref = O.block_scan(xs, dm, xp, R, z, D, base, 15, 14)
    hout = torch.full((B, D, N), 7, dtype=torch.int32, device="cuda")
    yo = ops.block_scan(T(xs), T(dm), T(xp), R, T(z), D, T(base), 15, 14, h_out=hout)
    assert np.array_equal(H(yo), yo_ref)
    assert np.array_equal(H(hout), h_ref)
