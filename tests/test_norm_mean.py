"""The norm's mean mu = floor(s1 / dim) is taken on the GPU as
floor(double(s1) / double(dim)) (csrc/mi_common.hpp, norm_shift_tab).  For
|s1| < 2^36 (|r| < 2^23 over dim <= 8192 features) the correctly rounded
double quotient is within 2^-17 of the exact one, which is either an integer
or at least 1/dim >= 2^-13 from one, so the floor is exact.  This checks that
claim with IEEE double division on the CPU: every integer quotient boundary
(k * dim and its neighbours) at the range ends, and random sums."""
import numpy as np


def _check(s1, dim):
    s1 = np.asarray(s1, dtype=np.int64)
    got = np.floor(s1.astype(np.float64) / np.float64(dim)).astype(np.int64)
    want = np.floor_divide(s1, dim)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (dim, s1[bad[:5]])


def test_mean_floor_at_quotient_boundaries():
    lim = (1 << 36) - 1
    for dim in (1, 2, 3, 7, 16, 255, 768, 1536, 2048, 4095, 4096, 8191, 8192):
        k_hi = lim // dim
        ks = np.concatenate([np.arange(-64, 65), np.arange(k_hi - 64, k_hi + 1), np.arange(-k_hi, -k_hi + 65)])
        base = ks.astype(np.int64) * dim
        s1 = np.concatenate([base - 1, base, base + 1])
        _check(s1[np.abs(s1) <= lim], dim)


def test_mean_floor_random_sums():
    rng = np.random.default_rng(5)
    lim = (1 << 36) - 1
    for dim in rng.integers(1, 8193, size=64):
        s1 = rng.integers(-lim, lim + 1, size=20000, dtype=np.int64)
        _check(s1, int(dim))
