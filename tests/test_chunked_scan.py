"""The chunked elementwise scan with ssd_chunked_scan_forward's outputs
(ssd_chunked_scan.py:382-422): h after every step, final_h at every chunk end,
decay_to_end as the chunk's Q30 cumulative decay.

CPU: the oracle's chunked form is pinned against the sequential elementwise
scan (brute force in Python integers and the oracle's own elementwise form),
final_h against h at the chunk ends, and decay_to_end against exact rational
products (closed forms at n = 2^k and n = 2^(k-1), and the bound
0 <= 2^30 * prod(n / 2^k) - p < steps for random decays).  GPU: the HIP
kernel against the oracle, bit for bit, through the C ABI and the drop-in.
"""
import ctypes
from fractions import Fraction

import numpy as np
import pytest

import oracle as O


def _inputs(rng, B, L, C, nlo=0, nhi=1 << 15, ulo=-(1 << 20), uhi=1 << 20):
    u = rng.integers(ulo, uhi, size=(B, L, C), dtype=np.int64).astype(np.int32)
    n = rng.integers(nlo, nhi + 1, size=(B, L, C), dtype=np.int64).astype(np.int32)
    return u, n


def _brute(u, n, k, h0=None):
    B, L, C = u.shape
    h = np.zeros((B, L, C), np.int64)
    for b in range(B):
        for c in range(C):
            s = 0 if h0 is None else int(h0[b, c])
            for t in range(L):
                s = max(-2**31, min(2**31 - 1, (s * int(n[b, t, c])) // (1 << k) + int(u[b, t, c])))
                h[b, t, c] = s
    return h


@pytest.mark.parametrize("chunk", [1, 3, 8, 13, 40, 41])
def test_oracle_h_is_the_sequential_scan(rng, chunk):
    u, n = _inputs(rng, 2, 40, 5)
    h0 = rng.integers(-2**24, 2**24, size=(2, 5), dtype=np.int32)
    h, fh, dte, hs = O.dyadic_chunked_scan(u, n, 15, chunk, h_state=h0)
    assert np.array_equal(h, _brute(u, n, 15, h0))
    assert np.array_equal(h, O.dyadic_scan_elementwise(u, n, 15, h_state=h0)[0])
    assert np.array_equal(hs, h[:, -1])
    ends = [min((c + 1) * chunk, 40) - 1 for c in range(-(-40 // chunk))]
    assert np.array_equal(fh, h[:, ends])


def test_oracle_saturates_h(rng):
    u = np.full((1, 6, 2), 2**31 - 1, np.int32)
    u[0, :, 1] = -2**31
    n = np.full((1, 6, 2), 1 << 15, np.int32)
    h, _, _ = O.dyadic_chunked_scan(u, n, 15, 4)
    assert (h[0, 1:, 0] == 2**31 - 1).all() and (h[0, 1:, 1] == -2**31).all()


def test_oracle_decay_to_end_closed_forms():
    """n = 2^k keeps 2^30; n = 2^(k-1) halves it exactly every step (chunk <= 30);
    n = 0 zeroes it; a ragged last chunk decays over its own steps only."""
    k = 15
    u = np.zeros((1, 70, 3), np.int32)
    n = np.zeros((1, 70, 3), np.int32)
    n[..., 0] = 1 << k
    n[..., 1] = 1 << (k - 1)
    _, _, dte = O.dyadic_chunked_scan(u, n, k, 25)
    assert dte.shape == (1, 3, 3)
    assert (dte[0, :, 0] == 1 << 30).all()
    assert dte[0, :, 1].tolist() == [1 << 5, 1 << 5, 1 << 10]      # chunks of 25, 25, 20 steps
    assert (dte[0, :, 2] == 0).all()


def test_oracle_decay_to_end_bounds_the_exact_product(rng):
    """With 0 <= n <= 2^k the floor-by-step product lies within `steps` units
    (Q30) below the exact rational product of the chunk's decays."""
    k, chunk = 15, 9
    u, n = _inputs(rng, 2, 30, 4, nlo=20000, nhi=1 << 15)
    _, _, dte = O.dyadic_chunked_scan(u, n, k, chunk)
    for b in range(2):
        for c in range(4):
            for ci in range(dte.shape[1]):
                steps = range(ci * chunk, min((ci + 1) * chunk, 30))
                exact = Fraction(1 << 30)
                for t in steps:
                    exact *= Fraction(int(n[b, t, c]), 1 << k)
                gap = exact - int(dte[b, ci, c])
                assert 0 <= gap < len(steps), (b, c, ci, float(gap))


def test_abi_validation():
    from mamba_int import _lib
    A = ctypes.c_void_p(0x100000)
    cases = [
        ((A, A, 15, 0, A, None, None, None, None, 1, 4, 4, None), 4, "chunk=0"),
        ((A, A, 31, 8, A, None, None, None, None, 1, 4, 4, None), 4, "decay_shift=31"),
        ((A, A, 15, 8, A, None, None, None, None, -1, 4, 4, None), 2, "negative"),
        ((None, A, 15, 8, A, None, None, None, None, 1, 4, 4, None), 1, "required"),
        ((A, A, 15, 8, None, None, None, None, None, 1, 4, 4, None), 1, "required"),
    ]
    for args, status, needle in cases:
        assert _lib.raw("mi_dyadic_chunked_scan", *args) == status, _lib.last_error()
        assert needle in _lib.last_error()
    assert _lib.raw("mi_dyadic_chunked_scan", None, None, 15, 8, None, None, None, None, None, 1, 0, 4, None) == 0


# ------------------------------------------------------------------ GPU
def _T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("B,L,C,chunk", [
    (2, 300, 100, 64), (1, 256, 8192, 64), (3, 97, 33, 1), (2, 50, 70, 256), (1, 1, 5, 64), (2, 129, 64, 8),
])
def test_gpu_chunked_scan_matches_oracle(cuda, B, L, C, chunk):
    """Ragged chunks, a chunk longer than the sequence, chunk 1, and the config-1
    scan flattened as the model feeds it ([1, 256, 512*16])."""
    from mamba_int import ops
    rng = np.random.default_rng(B * 7 + L + C + chunk)
    u, n = _inputs(rng, B, L, C)
    n[:, ::7] = 1 << 15                      # exact unit decays
    n[:, 3::11] = 0
    u[:, 5::13] = 2**31 - 1                  # saturation
    h_ref, fh_ref, dte_ref = O.dyadic_chunked_scan(u, n, 15, chunk)
    h, fh, dte = ops.dyadic_chunked_scan(_T(u), _T(n), 15, chunk)
    assert np.array_equal(h.cpu().numpy(), h_ref)
    assert np.array_equal(fh.cpu().numpy(), fh_ref)
    assert np.array_equal(dte.cpu().numpy(), dte_ref)


@pytest.mark.gpu
def test_gpu_chunked_scan_state_continuation_and_dropin(cuda):
    """Two calls with the state carried equal one call; the drop-in
    ssd_chunked_scan_forward returns the same three tensors."""
    import torch
    from mamba_int import ops
    from ssd_chunked_scan import SSDChunkedScanFunction, ssd_chunked_scan_forward
    rng = np.random.default_rng(3)
    u, n = _inputs(rng, 2, 200, 48, nlo=16384)
    h_ref, fh_ref, dte_ref = O.dyadic_chunked_scan(u, n, 12, 50)
    hs = torch.zeros((2, 48), dtype=torch.int32, device="cuda")
    h1, _, _ = ops.dyadic_chunked_scan(_T(u[:, :100]), _T(n[:, :100]), 12, 50, h_out=hs)
    h2, _, _ = ops.dyadic_chunked_scan(_T(u[:, 100:]), _T(n[:, 100:]), 12, 50, h_in=hs, h_out=hs)
    assert np.array_equal(np.concatenate([h1.cpu().numpy(), h2.cpu().numpy()], axis=1), h_ref)
    shifts = torch.full(u.shape, 12, dtype=torch.int32, device="cuda")
    h, fh, dte = ssd_chunked_scan_forward(_T(u), _T(n).to(torch.int64), shifts, 50)
    assert np.array_equal(h.cpu().numpy(), h_ref)
    assert np.array_equal(fh.cpu().numpy(), fh_ref)
    # the drop-in returns the reference's float32 decay_to_end: Q30 / 2^30
    assert dte.dtype == torch.float32
    assert np.array_equal(dte.cpu().numpy(), (dte_ref.astype(np.float32) / np.float32(2**30)))
    assert torch.equal(SSDChunkedScanFunction.apply(_T(u), _T(n), shifts, 50), h)
    with pytest.raises(ValueError):
        ssd_chunked_scan_forward(_T(u), _T(n), torch.tensor([12, 13], device="cuda"), 50)


@pytest.mark.gpu
@pytest.mark.parametrize("with_state", [True, False])
def test_gpu_scans_with_no_steps_carry_state(cuda, with_state):
    """len = 0 with h_out: no step runs and h_out receives h_in unchanged (zeros when
    h_in is None), for the chunked and the elementwise recurrence alike."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(12)
    B, C = 3, 70
    h0 = rng.integers(-2**31, 2**31, size=(B, C), dtype=np.int64).astype(np.int32)
    want = h0 if with_state else np.zeros_like(h0)
    u = torch.empty((B, 0, C), dtype=torch.int32, device="cuda")
    for run in ("chunked", "elementwise"):
        hs = torch.full((B, C), 0x5555, dtype=torch.int32, device="cuda")
        h_in = _T(h0) if with_state else None
        if run == "chunked":
            h, fh, dte = ops.dyadic_chunked_scan(u, u, 15, 8, h_in=h_in, h_out=hs)
            assert fh.shape == (B, 0, C) and dte.shape == (B, 0, C)
        else:
            h = ops.dyadic_scan_elementwise(u, u, 15, h_in=h_in, h_out=hs)
        assert h.shape == (B, 0, C)
        assert np.array_equal(hs.cpu().numpy(), want), run
