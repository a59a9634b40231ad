"""GPU parity of the scans against the CPU oracle (bit-exact)."""

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


def _scan_inputs(rng, B, L, D, N, nlo=16384, nhi=32767):
    x = i8(rng, B, L, D)
    b = i8(rng, B, L, N)
    c = i8(rng, B, L, N)
    n = rng.integers(nlo, nhi + 1, size=(D, N), dtype=np.int32)
    return x, b, c, n


def test_scan_config1_bit_exact(cuda):
    """Config 1: B1 L256 D512 N16, n ~ U[16384, 32767], k = 15."""
    from mamba_int import ops
    rng = np.random.default_rng(1)
    x, b, c, n = _scan_inputs(rng, 1, 256, 512, 16)
    hs = np.zeros((1, 512, 16), np.int32)
    y_ref, h_ref = O.dyadic_scan(x, b, c, n, 15, h_state=hs)
    h_out = T(hs)
    y = ops.dyadic_scan(T(x), T(b), T(c), T(n), 15, h_out=h_out)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(h_out), h_ref)


@pytest.mark.parametrize("B,L,D,N", [
    (2, 100, 64, 16), (1, 1, 16, 16), (3, 130, 48, 32), (2, 65, 128, 64),
    (1, 200, 32, 128), (1, 50, 40, 16), (2, 33, 32, 8), (1, 19, 16, 5),
    # the lane split G follows the channel count B*D at N = 16: 65536 channels
    # give G = 1, 32768 G = 2, 16384 G = 4, 8192 G = 8, fewer G = 16
    (2, 9, 32768, 16), (1, 11, 32768, 16), (1, 13, 16384, 16), (1, 21, 8192, 16), (2, 77, 64, 16),
])
def test_scan_shapes(cuda, B, L, D, N):
    """Fast kernel at every lane split, ragged D (generic path), odd N, odd L."""
    from mamba_int import ops
    rng = np.random.default_rng(B * 1000 + L * 10 + D + N)
    x, b, c, n = _scan_inputs(rng, B, L, D, N)
    y_ref = O.dyadic_scan(x, b, c, n, 15)
    y = ops.dyadic_scan(T(x), T(b), T(c), T(n), 15)
    assert np.array_equal(H(y), y_ref)


def test_scan_state_continuation(cuda):
    """Two calls with the carried state equal one call over the whole sequence."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(7)
    x, b, c, n = _scan_inputs(rng, 2, 300, 64, 16)
    y_ref = O.dyadic_scan(x, b, c, n, 15)
    h = torch.zeros((2, 64, 16), dtype=torch.int32, device="cuda")
    y1 = ops.dyadic_scan(T(x[:, :131]), T(b[:, :131]), T(c[:, :131]), T(n), 15, h_out=h)
    y2 = ops.dyadic_scan(T(x[:, 131:]), T(b[:, 131:]), T(c[:, 131:]), T(n), 15, h_in=h, h_out=h)
    assert np.array_equal(np.concatenate([H(y1), H(y2)], axis=1), y_ref)


def test_scan_extremes_saturation(cuda):
    """n = 2^k (pure accumulation) with maximal inputs drives h into int32 saturation."""
    from mamba_int import ops
    B, L, D, N = 1, 64, 16, 16
    x = np.full((B, L, D), 127, np.int8)
    b = np.full((B, L, N), 127, np.int8)
    c = np.full((B, L, N), -128, np.int8)
    n = np.full((D, N), 1 << 15, np.int32)
    h0 = np.full((B, D, N), 2**31 - 100000, np.int32)
    y_ref, h_ref = O.dyadic_scan(x, b, c, n, 15, h_state=h0)
    hin = T(h0)
    hout = T(np.zeros_like(h0))
    y = ops.dyadic_scan(T(x), T(b), T(c), T(n), 15, h_in=hin, h_out=hout)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(hout), h_ref)
    assert (h_ref == 2**31 - 1).all()


def test_scan_k16_and_generic_shift(cuda):
    from mamba_int import ops
    rng = np.random.default_rng(3)
    for k, nhi in ((16, 65536), (12, 4096), (1, 2)):
        x, b, c, n = _scan_inputs(rng, 2, 70, 32, 16, nlo=0, nhi=nhi)
        y_ref = O.dyadic_scan(x, b, c, n, k)
        y = ops.dyadic_scan(T(x), T(b), T(c), T(n), k)
        assert np.array_equal(H(y), y_ref), k


def test_scan_f32_reference_semantics(cuda):
    """mi_dyadic_scan_f32 = the reference launch_dyadic_scan (int64 state, fp32 I/O)."""
    from mamba_int import ops
    rng = np.random.default_rng(5)
    B, S, D = 2, 100, 256
    x = rng.standard_normal((B, S, D)).astype(np.float32)
    nums = rng.integers(20000, 32000, size=(B, S, D), dtype=np.int32)
    shifts = np.full((B, S, D), 15, np.int32)
    h_ref = O.dyadic_scan_f32(x, nums, shifts, 20)
    h = ops.dyadic_scan_f32(T(x), T(nums), T(shifts), 20)
    assert np.array_equal(H(h).view(np.uint32), h_ref.view(np.uint32))


@pytest.mark.parametrize("sb", [0, 8, 20, 40])
def test_scan_f32_varied_shifts_and_scale_bits(cuda, sb):
    """Per-element shifts in {0, 1, 7, 15, 31} with nums up to 2^shift, signs and
    magnitudes mixed, plus exact fractional inputs (-1.5, 1.75, -0.25 units: truncation
    toward zero) and a negative impulse at decay 1/2 (arithmetic-shift floor); the
    inputs keep |h * num| < 2^63 as the reference's int64 state requires."""
    from mamba_int import ops
    rng = np.random.default_rng(50 + sb)
    B, S, D = 3, 96, 200
    mag = rng.choice([0.5, 4.0, 16.0], size=(B, S, D)) * (2.0 ** -max(0, sb - 20))
    x = (rng.standard_normal((B, S, D)) * mag).astype(np.float32)
    shifts = rng.choice(np.array([0, 1, 7, 15, 31], np.int32), size=(B, S, D)).astype(np.int32)
    hi = np.minimum(np.left_shift(np.int64(1), shifts.astype(np.int64)), 2**31 - 1)
    nums = (rng.random((B, S, D)) * (hi + 1)).astype(np.int64).clip(0, 2**31 - 1).astype(np.int32)
    nums[shifts == 0] = rng.integers(0, 2, size=int((shifts == 0).sum()))   # decay 0 or 1
    u = 2.0 ** -sb
    x[0, :, 0] = np.float32(-1.5 * u)
    x[0, :, 1] = np.float32(1.75 * u)
    x[0, :, 2] = np.float32(-0.25 * u)
    nums[0, :, :3] = 0
    x[1, :, 3] = 0
    x[1, 0, 3] = np.float32(-3 * u)
    nums[1, :, 3], shifts[1, :, 3] = 1, 1
    assert (np.abs(x.astype(np.float64)) * 2.0 ** sb).sum(axis=1).max() * 2**31 < 2**63
    h_ref = O.dyadic_scan_f32(x, nums, shifts, sb)
    h = H(ops.dyadic_scan_f32(T(x), T(nums), T(shifts), sb))
    assert np.array_equal(h.view(np.uint32), h_ref.view(np.uint32))
    assert np.array_equal(h[0, :, :3].astype(np.float64) / u,
                          np.tile([-1.0, 1.0, 0.0], (S, 1)))
    assert np.array_equal(h[1, :5, 3].astype(np.float64) / u, [-3, -2, -1, -1, -1])


def test_scan_elementwise(cuda):
    from mamba_int import ops
    rng = np.random.default_rng(9)
    B, L, C = 2, 90, 300
    u = rng.integers(-2**20, 2**20, size=(B, L, C), dtype=np.int32)
    nn = rng.integers(0, 32768, size=(B, L, C), dtype=np.int32)
    h_ref = O.dyadic_scan_elementwise(u, nn, 15)
    h = ops.dyadic_scan_elementwise(T(u), T(nn), 15)
    assert np.array_equal(H(h), h_ref)


@pytest.mark.parametrize("B,L,H_,P,N,cs", [
    (2, 512, 3, 64, 128, 256), (1, 300, 2, 64, 128, 64), (1, 130, 2, 32, 64, 100), (2, 64, 1, 16, 16, 64),
])
def test_ssd_chunked(cuda, B, L, H_, P, N, cs):
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(L + H_ + P + N)
    x = i8(rng, B, L, H_, P)
    b = i8(rng, B, L, H_, N)
    c = i8(rng, B, L, H_, N)
    n = rng.integers(24576, 32768, size=(H_,), dtype=np.int32)
    y_ref, cst_ref, h_ref = O.ssd_chunked_scan(x, b, c, n, 15, cs, want_chunk_states=True,
                                               h_state=np.zeros((B, H_, P, N), np.int32))
    nc = -(-L // cs)
    cst = torch.zeros((B, nc, H_, P, N), dtype=torch.int32, device="cuda")
    hout = torch.zeros((B, H_, P, N), dtype=torch.int32, device="cuda")
    y = ops.ssd_chunked_scan(T(x), T(b), T(c), T(n), 15, cs, chunk_states=cst, h_out=hout)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(cst), cst_ref)
    assert np.array_equal(H(hout), h_ref)


@pytest.mark.parametrize("B,L,H_,P,cs", [(2, 203, 48, 64, 64), (8, 192, 32, 24, 128), (1, 130, 96, 64, 64)])
def test_ssd_chunked_mixed_block(cuda, B, L, H_, P, cs):
    """N = 128 shapes whose 24-channel blocks fill 256 CUs exactly: the mixed
    block (16- and 32-lane waves; blocks straddling two heads, the last head's
    block without a neighbour, one head per block at P = 24), a ragged last
    chunk (L = 203, 130: the 1-3 step tail), chunk states at every cs and at
    the end, and a nonzero start state."""
    import torch
    from mamba_int import ops
    N = 128
    rng = np.random.default_rng(B * L + H_ + P)
    x = i8(rng, B, L, H_, P)
    b = i8(rng, B, L, H_, N)
    c = i8(rng, B, L, H_, N)
    n = rng.integers(24576, 32768, size=(H_,), dtype=np.int32)
    h0 = rng.integers(-(2**31), 2**31, size=(B, H_, P, N), dtype=np.int64).astype(np.int32)
    y_ref, cst_ref, h_ref = O.ssd_chunked_scan(x, b, c, n, 15, cs, want_chunk_states=True, h_state=h0.copy())
    nc = -(-L // cs)
    cst = torch.zeros((B, nc, H_, P, N), dtype=torch.int32, device="cuda")
    hout = torch.zeros((B, H_, P, N), dtype=torch.int32, device="cuda")
    y = ops.ssd_chunked_scan(T(x), T(b), T(c), T(n), 15, cs, chunk_states=cst, h_in=T(h0), h_out=hout)
    assert np.array_equal(H(y), y_ref)
    assert np.array_equal(H(cst), cst_ref)
    assert np.array_equal(H(hout), h_ref)


def test_ssd_config4_full_size(cuda):
    """Config 4 at full size (B4 L8192 H24 P64 N128, cs 256) on the GPU against
    the oracle, bit for bit: every output, every chunk-boundary state and the
    final state (6.4 G state updates; the oracle takes a few seconds)."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(4)
    B, L, H_, P, N = 4, 8192, 24, 64, 128
    x = i8(rng, B, L, H_, P)
    b = i8(rng, B, L, H_, N)
    c = i8(rng, B, L, H_, N)
    n = rng.integers(24576, 32768, size=(H_,), dtype=np.int32)
    nc = L // 256
    cs = torch.empty((B, nc, H_, P, N), dtype=torch.int32, device="cuda")
    hout = torch.empty((B, H_, P, N), dtype=torch.int32, device="cuda")
    y = H(ops.ssd_chunked_scan(T(x), T(b), T(c), T(n), 15, 256, chunk_states=cs, h_out=hout))
    hs = np.zeros((B, H_, P, N), np.int32)
    y_ref, cs_ref, hs_ref = O.ssd_chunked_scan(x, b, c, n, 15, 256, want_chunk_states=True, h_state=hs)
    assert np.array_equal(y, y_ref)
    assert np.array_equal(H(cs), cs_ref)
    assert np.array_equal(H(hout), hs_ref)


def test_ssd_equals_channel_scan(cuda):
    """Per head, the chunked multi-head scan equals the config-1 scan with a constant decay."""
    from mamba_int import ops
    rng = np.random.default_rng(11)
    B, L, H_, P, N = 1, 256, 2, 64, 64
    x = i8(rng, B, L, H_, P)
    b = i8(rng, B, L, H_, N)
    c = i8(rng, B, L, H_, N)
    n = rng.integers(24576, 32768, size=(H_,), dtype=np.int32)
    y = H(ops.ssd_chunked_scan(T(x), T(b), T(c), T(n), 15, 128))
    for hd in range(H_):
        yc = H(ops.dyadic_scan(T(np.ascontiguousarray(x[:, :, hd])), T(np.ascontiguousarray(b[:, :, hd])),
                               T(np.ascontiguousarray(c[:, :, hd])), T(np.full((P, N), n[hd], np.int32)), 15))
        assert np.array_equal(y[:, :, hd], yc)
