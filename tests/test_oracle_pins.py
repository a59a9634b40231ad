"""Pins of the CPU oracle against what the reference and the mathematics fix.

The reference ships no golden vectors (its tests print numbers); each oracle
function is pinned here by an independent route: closed forms of the
recurrence, brute force with Python integers, the reference's own torch ops on
the CPU (F.linear, torch.round, conv1d), exact rationals for the threshold
table, math.isqrt for the square roots.  test_mutations_are_caught plants a
mistake in the oracle and shows the pins fail.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from conftest import i8


# ------------------------------------------------------------------ scans
def _py_scan(x, b, c, n, k, h0=None):
    """Brute force with Python integers: floor via //, saturation as stated."""
    B, L, D = x.shape
    N = b.shape[-1]
    y = np.zeros((B, L, D), np.int64)
    hs = np.zeros((B, D, N), np.int64) if h0 is None else h0.astype(np.int64).copy()
    for bb in range(B):
        for d in range(D):
            h = [int(v) for v in hs[bb, d]]
            for t in range(L):
                acc = 0
                for j in range(N):
                    v = (h[j] * int(n[d, j])) // (1 << k) + int(b[bb, t, j]) * int(x[bb, t, d])
                    h[j] = max(-2**31, min(2**31 - 1, v))
                    acc += int(c[bb, t, j]) * h[j]
                y[bb, t, d] = max(-2**31, min(2**31 - 1, acc))
            hs[bb, d] = h
    return y, hs


def test_scan_brute_force(rng):
    x, b, c = i8(rng, 2, 23, 5), i8(rng, 2, 23, 6), i8(rng, 2, 23, 6, lo=-128)
    n = rng.integers(0, 2**15 + 1, size=(5, 6), dtype=np.int32)
    h0 = rng.integers(-2**31, 2**31, size=(2, 5, 6), dtype=np.int64).astype(np.int32)
    y, hs = O.dyadic_scan(x, b, c, n, 15, h_state=h0)
    y2, hs2 = _py_scan(x, b, c, n, 15, h0)
    assert np.array_equal(y, y2) and np.array_equal(hs, hs2)


def test_scan_closed_form_full_decay_is_prefix_sum(rng):
    """n = 2^k: h_t = sum_{s<=t} B_s x_s (no saturation at these sizes)."""
    x, b, c = i8(rng, 2, 300, 7), i8(rng, 2, 300, 4), i8(rng, 2, 300, 4)
    n = np.full((7, 4), 1 << 15, np.int32)
    h = np.cumsum(b[:, :, None, :].astype(np.int64) * x[:, :, :, None], axis=1)   # [B,L,D,N]
    y_ref = np.einsum("bln,bldn->bld", c.astype(np.int64), h)
    assert np.array_equal(O.dyadic_scan(x, b, c, n, 15), y_ref)


def test_scan_closed_form_zero_decay(rng):
    """n = 0: h_t = u_t, so y_t = sum_n C_t B_t x_t (keeps the input's sign)."""
    x, b, c = i8(rng, 1, 50, 9), i8(rng, 1, 50, 8), i8(rng, 1, 50, 8)
    n = np.zeros((9, 8), np.int32)
    y_ref = np.einsum("bln,bln,bld->bld", c.astype(np.int64), b.astype(np.int64), x.astype(np.int64))
    assert np.array_equal(O.dyadic_scan(x, b, c, n, 15), y_ref)


def test_scan_impulse_floor_semantics():
    """Decay 1/2 (n = 2^14, k = 15) on impulses u_0 = +-128: +128 halves to 0 after
    8 steps; -128 halves to -1 and stays there (floor(-1/2) = -1, the arithmetic
    shift of dyadic_mamba_kernel.cu:56)."""
    L = 12
    for sign in (1, -1):
        x = np.zeros((1, L, 1), np.int8)
        x[0, 0, 0] = 2 * sign
        b = np.full((1, L, 1), 64, np.int8)
        c = np.ones((1, L, 1), np.int8)
        n = np.full((1, 1), 1 << 14, np.int32)
        y = O.dyadic_scan(x, b, c, n, 15)[0, :, 0]
        if sign > 0:
            expect = [128 >> t for t in range(L)]
        else:
            expect = [-(128 >> t) if t < 8 else -1 for t in range(L)]
        assert y.tolist() == expect


def test_scan_y_saturates_once():
    """Partial sums C*h exceed int32 but their total is 0: y must be 0."""
    x = np.zeros((1, 1, 1), np.int8)
    b = np.zeros((1, 1, 2), np.int8)
    c = np.array([[[127, -127]]], np.int8)
    n = np.full((1, 2), 1 << 15, np.int32)
    h0 = np.full((1, 1, 2), 2**30, np.int32)
    assert O.dyadic_scan(x, b, c, n, 15, h_state=h0)[0][0, 0, 0] == 0


def test_scan_state_bound(rng):
    """|h_t| <= |h_0| + sum |u| for 0 <= n <= 2^k."""
    x, b, c = i8(rng, 1, 200, 3), i8(rng, 1, 200, 5), i8(rng, 1, 200, 5)
    n = rng.integers(0, 2**15 + 1, size=(3, 5), dtype=np.int32)
    h0 = rng.integers(-2**20, 2**20, size=(1, 3, 5)).astype(np.int32)
    cst = O.ssd_chunked_scan(x[:, :, None, :], b[:, :, None, :], c[:, :, None, :],
                             np.array([n[0, 0]], np.int32), 15, 200, want_chunk_states=True,
                             h_state=np.repeat(h0[:, None, :, :1], 1, axis=1).reshape(1, 1, 3, 1)
                             .repeat(5, axis=3))[1]
    bound = np.abs(h0[0, :, :1]).astype(np.int64).repeat(5, 1) + \
        np.sum(np.abs(b[0, :, None, :].astype(np.int64) * x[0, :, :, None]), axis=0)
    assert np.all(np.abs(cst[0, 0, 0].astype(np.int64)) <= bound)


def test_scan_f32_matches_reference_python_forward(rng):
    """Reference kernel form vs the reference's fp64 simulation (test_mamba_scan.py:45-67):
    the kernel floors each step in 2^-sb units, so it lies below the fp64 value by less
    than (t+2) units, plus fp32 output rounding."""
    B, S, D, sb = 1, 100, 64, 20
    x = rng.standard_normal((B, S, D)).astype(np.float32)
    nums = rng.integers(20000, 32000, size=(B, S, D), dtype=np.int32)
    shifts = np.full((B, S, D), 15, np.int32)
    hk = O.dyadic_scan_f32(x, nums, shifts, sb).astype(np.float64)
    h = np.zeros((B, D))
    for t in range(S):
        h = h * (nums[:, t] / 2.0**shifts[:, t]) + x[:, t].astype(np.float64) * 2.0**sb
        hp = h / 2.0**sb
        tol = (t + 2) * 2.0**-sb + np.abs(hp) * 2.0**-23
        diff = hp - hk[:, t]
        assert np.all(diff >= -tol) and np.all(diff <= tol)


# Exact pins of the float-compat scan (dyadic_mamba_kernel.cu:35-63).  The kernel's
# float steps are exact except two: x * 2^sb is a power-of-two scaling (exact in fp32),
# the conversion to long long truncates toward zero, (float)h rounds to nearest-even,
# and the division by 2^sb is exact again.  So the whole output is fixed by integer
# arithmetic plus one rounding, restated here with Python integers.
def _f32_round_int(h: int) -> int:
    """The integer value of (float)h: round to 24 significant bits, ties to even."""
    a = abs(h)
    drop = a.bit_length() - 24
    if drop <= 0:
        return h
    q, r = a >> drop, a & ((1 << drop) - 1)
    half = 1 << (drop - 1)
    if r > half or (r == half and q & 1):
        q += 1
    return (q << drop) * (1 if h >= 0 else -1)


def _py_scan_f32(x, nums, shifts, sb):
    """Brute force of launch_dyadic_scan with Python integers; output in float64
    (every value it takes is exact there: 24-bit significand times a power of 2)."""
    B, S, D = x.shape
    out = np.zeros((B, S, D), np.float64)
    for b in range(B):
        for d in range(D):
            h = 0
            for t in range(S):
                xf = math.trunc(Fraction(float(x[b, t, d])) * (1 << sb))   # toward zero
                h = (h * int(nums[b, t, d])) >> int(shifts[b, t, d])      # Python >> floors
                h += xf
                out[b, t, d] = _f32_round_int(h) / 2.0**sb
    return out


def _f32_exact(hk, want):
    return np.array_equal(hk.astype(np.float64), want)


def test_f32_round_int_known_values():
    """(float) of integers at the rounding boundaries of a 24-bit significand."""
    assert _f32_round_int(2**24 + 1) == 2**24                 # tie, even stays
    assert _f32_round_int(2**24 + 3) == 2**24 + 4             # tie, odd rounds up
    assert _f32_round_int(-(2**24 + 3)) == -(2**24 + 4)
    assert _f32_round_int(2**25 + 3) == 2**25 + 4             # above half
    assert _f32_round_int(2**25 + 1) == 2**25
    # against the hardware's float64 -> float32 conversion (each v is exact in float64)
    for v in (2**24 + 1, 2**24 + 3, 2**25 + 3, 2**40 + 2**16 + 1, -(2**33 + 2**9), 2**40 + 2**16):
        assert _f32_round_int(v) == int(np.float32(float(v))), v


def test_scan_f32_truncates_toward_zero():
    """num = 0 leaves h = x_fixed = trunc(x * 2^sb): -1.5 units gives -1 (floor gives -2,
    round gives -2), +1.75 units gives 1 (round gives 2), -0.25 units gives 0."""
    for sb in (0, 8, 20):
        u = 2.0**-sb
        vals = np.array([-1.5, 1.75, -0.25, 0.75, -2.5, 3.5, -1000.75, 123456.5], np.float64) * u
        x = vals.astype(np.float32).reshape(1, -1, 1)
        assert np.array_equal(x.astype(np.float64).ravel(), vals)        # exact inputs
        nums = np.zeros(x.shape, np.int32)
        shifts = np.full(x.shape, 15, np.int32)
        hk = O.dyadic_scan_f32(x, nums, shifts, sb)
        want = np.array([-1, 1, 0, 0, -2, 3, -1000, 123456], np.float64) * u
        assert np.array_equal(hk.astype(np.float64).ravel(), want), sb


def test_scan_f32_full_decay_is_prefix_sum(rng):
    """num = 2^shift: h_t = sum of trunc(x_s * 2^sb), output (float)h_t / 2^sb."""
    for sb, shift in ((20, 15), (8, 7), (0, 1), (12, 30)):
        x = (rng.standard_normal((2, 60, 9)) * 3).astype(np.float32)
        nums = np.full(x.shape, 1 << shift, np.int32)
        shifts = np.full(x.shape, shift, np.int32)
        xf = np.trunc(x.astype(np.float64) * 2.0**sb).astype(np.int64)
        pref = np.cumsum(xf, axis=1)
        want = np.vectorize(lambda v: float(_f32_round_int(int(v))))(pref) / 2.0**sb
        assert _f32_exact(O.dyadic_scan_f32(x, nums, shifts, sb), want), (sb, shift)


def test_scan_f32_negative_impulse_floors():
    """Decay 1/2 on a negative state: the arithmetic shift floors, so -3 -> -2 -> -1 -> -1
    and stays there (a truncating divide would reach 0); a positive impulse 3 -> 1 -> 0."""
    for sb in (0, 8, 20):
        x = np.zeros((1, 6, 2), np.float32)
        x[0, 0, 0] = np.float32(-3 * 2.0**-sb)
        x[0, 0, 1] = np.float32(3 * 2.0**-sb)
        for num, shift in ((1, 1), (64, 7), (1 << 14, 15), (1 << 30, 31)):
            nums = np.full(x.shape, num, np.int32)
            shifts = np.full(x.shape, shift, np.int32)
            hk = O.dyadic_scan_f32(x, nums, shifts, sb).astype(np.float64) * 2.0**sb
            assert np.array_equal(hk[0, :, 0], [-3, -2, -1, -1, -1, -1]), (sb, num, shift)
            assert np.array_equal(hk[0, :, 1], [3, 1, 0, 0, 0, 0]), (sb, num, shift)


def test_scan_f32_output_rounds_to_nearest_even():
    """(float)h on states above 2^24 (num 1, shift 0: no decay; sb 0): step 0 loads
    2^24, 2^24, 2^25, -2^24; step 1 adds 1, 3, 3, -3.  2^24 + 1 and 2^24 + 3 are ties
    (even significand wins), 2^25 + 3 lies above the half."""
    x = np.array([[[2**24, 2**24, 2**25, -2**24], [1, 3, 3, -3]]], np.float32)
    nums = np.ones(x.shape, np.int32)
    shifts = np.zeros(x.shape, np.int32)
    hk = O.dyadic_scan_f32(x, nums, shifts, 0).astype(np.float64)
    assert np.array_equal(hk[0, 1], [2**24, 2**24 + 4, 2**25 + 4, -(2**24 + 4)])


@pytest.mark.parametrize("sb", [0, 8, 20])
def test_scan_f32_brute_force(rng, sb):
    """Random inputs, per-element shifts in {1, 7, 15, 31} with nums up to 2^shift, mixed
    signs and magnitudes: equal to the Python-integer brute force at every step."""
    B, S, D = 2, 40, 6
    x = (rng.standard_normal((B, S, D)) * rng.choice([0.5, 4.0, 16.0], size=(B, S, D)))
    x = x.astype(np.float32)
    # inside the reference's defined range: |h * num| < 2^63 with |h| <= sum |x_fixed|
    assert (np.abs(x.astype(np.float64)) * 2.0**sb).sum(axis=1).max() * 2**31 < 2**63
    shifts = rng.choice(np.array([1, 7, 15, 31], np.int32), size=(B, S, D)).astype(np.int32)
    hi = np.minimum(np.left_shift(np.int64(1), shifts.astype(np.int64)), 2**31 - 1)
    nums = (rng.random((B, S, D)) * (hi + 1)).astype(np.int64).clip(0, 2**31 - 1).astype(np.int32)
    hk = O.dyadic_scan_f32(x, nums, shifts, sb)
    assert _f32_exact(hk, _py_scan_f32(x, nums, shifts, sb))


def test_ssd_chunked_equals_sequential_for_any_chunk(rng):
    B, L, H, P, N = 2, 97, 3, 8, 16
    x, b, c = i8(rng, B, L, H, P), i8(rng, B, L, H, N), i8(rng, B, L, H, N)
    n = rng.integers(24576, 32768, size=(H,), dtype=np.int32)
    ys = []
    for hd in range(H):
        ys.append(O.dyadic_scan(x[:, :, hd], b[:, :, hd], c[:, :, hd], np.full((P, N), n[hd], np.int32), 15))
    seq = np.stack(ys, axis=2)
    for cs in (1, 7, 64, 97, 256):
        y, cst = O.ssd_chunked_scan(x, b, c, n, 15, cs, want_chunk_states=True)
        assert np.array_equal(y, seq), cs
        for ci in range(cst.shape[1]):
            tend = min(L, (ci + 1) * cs)
            _, hs = O.ssd_chunked_scan(x[:, :tend], b[:, :tend], c[:, :tend], n, 15, 1 << 20,
                                       h_state=np.zeros((B, H, P, N), np.int32))
            assert np.array_equal(cst[:, ci], hs)


def test_elementwise_scan_is_the_reference_op(rng):
    """DyadicScanFunction layout [B, L, D*N]: brute force with Python integers."""
    u = rng.integers(-2**24, 2**24, size=(2, 30, 11), dtype=np.int32)
    nn = rng.integers(0, 2**15 + 1, size=(2, 30, 11), dtype=np.int32)
    h = O.dyadic_scan_elementwise(u, nn, 15)
    ref = np.zeros_like(h)
    for bb in range(2):
        for ch in range(11):
            s = 0
            for t in range(30):
                s = max(-2**31, min(2**31 - 1, (s * int(nn[bb, t, ch])) // 32768 + int(u[bb, t, ch])))
                ref[bb, t, ch] = s
    assert np.array_equal(h, ref)


# ----------------------------------------------------------------- ternary
def test_pack_roundtrip_and_layout(rng):
    from mamba_int import pack_ternary, unpack_ternary
    w = rng.integers(-1, 2, size=(33, 64), dtype=np.int8)
    p = O.pack_ternary(w)
    assert np.array_equal(O.unpack_ternary(p, 64), w)
    assert np.array_equal(pack_ternary(w), p)
    assert np.array_equal(unpack_ternary(p, 64), w)
    # layout: weight 16w+4j+i at bits [8i+2j, 8i+2j+1] of little-endian word w
    one = np.zeros((1, 16), np.int8)
    one[0, 4 * 2 + 1] = -1           # j = 2, i = 1 -> bits 12..13 = 0b11
    one[0, 4 * 3 + 0] = 1            # j = 3, i = 0 -> bits 6..7 = 0b01
    word = int.from_bytes(bytes(O.pack_ternary(one)[0]), "little")
    assert word == (0b11 << 12) | (0b01 << 6)


def test_pack_all_81_patterns():
    import itertools
    pats = np.array(list(itertools.product((-1, 0, 1), repeat=4)), np.int8)   # 81 x 4
    w = np.zeros((81, 16), np.int8)
    for pos in range(4):
        w[:, 4 * pos:4 * pos + 4] = np.roll(pats, pos, axis=0)
    assert np.array_equal(O.unpack_ternary(O.pack_ternary(w), 16), w)


def test_bitlinear_equals_reference_f_linear(rng):
    """int32 accumulate == F.linear on integer-valued fp32 (rational_bitnet.py:204), exact
    because |sum| <= K*127 < 2^24."""
    M, K, N = 37, 768, 70
    a = i8(rng, M, K)
    w = rng.integers(-1, 2, size=(N, K), dtype=np.int8)
    acc = O.bitlinear(a, O.pack_ternary(w), O.OUT_INT32)
    ref = F.linear(torch.from_numpy(a).float(), torch.from_numpy(w).float()).numpy()
    assert np.array_equal(acc, ref.astype(np.int64))
    for s in (0, 1, 5):
        q = O.bitlinear(a, O.pack_ternary(w), O.OUT_INT8, s)
        expect = np.clip(np.floor(ref / 2**s + 0.5), -127, 127) if s else np.clip(ref, -127, 127)
        assert np.array_equal(q, expect.astype(np.int8))
    dm = O.bitlinear(a, O.pack_ternary(w), O.OUT_DECAY_MOD, 6)
    assert np.array_equal(dm, np.clip(np.floor(ref / 64 + 0.5), -20, 20).astype(np.int8))
    r0 = rng.integers(-2**23 + 1, 2**23, size=(M, N), dtype=np.int32)
    r = O.bitlinear(a, O.pack_ternary(w), O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16)
    expect = np.clip(r0 + np.floor(ref.astype(np.float64) * 4719 / 65536 + 0.5), -(2**23 - 1), 2**23 - 1)
    assert np.array_equal(r, expect.astype(np.int32))
    # the SSD block's out clamp: clamp(out_proj(y), -100, 100) before the residual gate
    # (ssd_multihead.py:589-590), on the accumulator: +-c, then the same residual rule
    for c in (1, 300, 2000):
        assert (np.abs(ref) > c).any()
        r = O.bitlinear(a, O.pack_ternary(w), O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16, res_clamp=c)
        expect = np.clip(r0 + np.floor(np.clip(ref.astype(np.float64), -c, c) * 4719 / 65536 + 0.5),
                         -(2**23 - 1), 2**23 - 1)
        assert np.array_equal(r, expect.astype(np.int32)), c


def test_act_quant_matches_reference_torch(rng):
    """activation_quant_dynamic (rational_bitnet.py:102-111) with torch on the CPU,
    including exact .5 ties (torch.round is half-to-even)."""
    x = torch.from_numpy(rng.standard_normal((40, 96)).astype(np.float32))
    x[0, :6] = torch.tensor([127.0, 0.5, -0.5, 1.5, 2.5, -2.5])        # amax 127: x*inv = x exactly
    x[1, :3] = torch.tensor([0.0, 0.0, 0.0])
    x[2] = 0.0
    sc = torch.amax(torch.abs(x), dim=-1, keepdim=True).clamp(min=1e-8)
    xq = torch.round(x * (127 / sc)).clamp(-127, 127)
    q, s = O.act_quant_f32(x.numpy())
    assert np.array_equal(q, xq.numpy().astype(np.int8))
    assert np.array_equal(s.view(np.uint32), (sc / 127).reshape(-1).numpy().view(np.uint32))
    assert q[0, :6].tolist() == [127, 0, 0, 2, 2, -2]
    y = O.bitlinear(q, O.pack_ternary(np.ones((3, 96), np.int8)), O.OUT_FLOAT, x_scale=s, w_scale=0.37)
    ref = F.linear(xq, torch.ones(3, 96)) * (torch.tensor(0.37) * (sc / 127))
    assert np.array_equal(y.view(np.uint32), ref.numpy().view(np.uint32))


# ------------------------------------------------------------------- norm
def _ref_table_k(var: Fraction) -> int:
    """The threshold cascade of _find_power_of_2_scale (mamba_integer_model.py:165-182),
    evaluated on an exact rational var, returned as the exponent k of scale = 2^-k."""
    scale = Fraction(1)
    for j, th in enumerate((4, 16, 64, 256, 1024, 4096, 16384, 65536), start=1):
        if var >= th:
            scale = Fraction(1, 2**j)
    if var < 1:
        scale = Fraction(1)
    for v, th in ((2, Fraction(1, 4)), (4, Fraction(1, 16)), (8, Fraction(1, 64))):
        if var < th:
            scale = Fraction(v)
    return -int(math.log2(scale))


def _py_norm(r, gamma):
    d = r.shape[-1]
    out = np.zeros(r.shape, np.int8)
    for t in range(r.shape[0]):
        row = [int(v) for v in r[t]]
        mu = sum(row) // d
        xs = [v - mu for v in row]
        k = _ref_table_k(Fraction(sum(v * v for v in xs), d * 2**16))
        sh = 12 + k
        for i in range(d):
            out[t, i] = max(-127, min(127, (xs[i] * int(gamma[i]) + (1 << (sh - 1))) >> sh))
    return out


def test_norm_table_and_rounding(rng):
    d = 48
    rows = [rng.integers(-2**23 + 1, 2**23, size=d), rng.integers(-5, 6, size=d), np.zeros(d, np.int64),
            rng.integers(-300, 300, size=d), -np.arange(d) * 7 - 3]
    # rows whose S = sum x^2 sits exactly on a threshold d*4^(j+8) or one below it
    for j in (1, 3, 5, 8, -1, -2, -3):
        target = d * 4 ** (j + 8) if j > 0 else d * 4 ** (8 + j)
        v = math.isqrt(target // d)
        row = np.zeros(d, np.int64)
        row[: d // 2] = v
        row[d // 2:] = -v
        rows.append(row)
        rows.append(row + np.where(np.arange(d) == 0, 1, 0))
    r = np.array(rows, np.int32)
    g = rng.integers(-400, 400, size=d, dtype=np.int16)
    g[0] = 256
    assert np.array_equal(O.bitshift_norm(r, g), _py_norm(r, g))


# ------------------------------------------------ squareplus / dt / gate
def test_squareplus_exact_and_close_to_float():
    for c in list(range(-52000, 52001, 7)) + [-51200, 51200, 0, 1, -1, 10**6, -10**6]:
        v = max(-51200, min(51200, c))
        exact = max(-127, min(127, (v + math.isqrt(v * v + 2**22) + 64) >> 7))
        got = O.squareplus_q(c)
        assert got == exact
        xf = v / 1024.0
        fl = 0.5 * (xf + math.sqrt(xf * xf + 4.0)) * 16
        assert abs(got - min(fl, 127.0)) <= 0.5 + 1e-9 or got == 127


def test_dt_table():
    for dm in range(-20, 21):
        s = dm * 65536 + math.isqrt(dm * dm * 2**32 + 2**34)
        sq = s >> 1
        exact = max(66, min(6554, (655 * sq + 2**15) >> 16))
        assert O.dt_q16(dm) == exact
        fl = min(0.1, max(0.001, 0.5 * (dm + math.sqrt(dm * dm + 4)) * 0.01)) * 65536
        # 655/2^16 = 0.0099945 stands for 0.01: relative error 5.5e-4, plus one unit of rounding
        assert abs(O.dt_q16(dm) - fl) <= 1 + 0.0006 * fl


def test_gate_table():
    for z in range(-128, 128):
        a = abs(z)
        q = (16384 * a) // (16 + a)
        assert O.gate_q15(z) == 16384 + (q if z >= 0 else -q)
        zf = z / 16.0
        assert abs(O.gate_q15(z) / 32768 - (0.5 + 0.5 * zf / (1 + abs(zf)))) < 2.0 / 32768


# ------------------------------------------------------------------- conv
@pytest.mark.parametrize("L", [1, 2, 3, 40])
def test_conv_squareplus_matches_reference_conv1d(rng, L):
    """Depthwise causal conv = nn.Conv1d(k=4, groups=D, padding=3)[..., :L]
    (mamba_integer_model.py:378,404) in float64 (exact on these integers)."""
    B, D = 2, 24
    xz = i8(rng, B, L, 2 * D)
    w = i8(rng, D, 4)
    bias = rng.integers(-60000, 60000, size=D, dtype=np.int32)
    xs, st = O.conv_squareplus(xz, D, w, bias)
    xin = torch.from_numpy(xz[:, :, :D].astype(np.float64)).transpose(1, 2)
    conv = F.conv1d(xin, torch.from_numpy(w.astype(np.float64))[:, None, :],
                    torch.from_numpy(bias.astype(np.float64)), padding=3, groups=D)[:, :, :L]
    c = conv.transpose(1, 2).numpy().astype(np.int64)
    expect = np.vectorize(O.squareplus_q)(c)
    assert np.array_equal(xs, expect)
    full = np.concatenate([np.zeros((B, 3, D), np.int8), xz[:, :, :D]], axis=1)
    assert np.array_equal(st, full[:, -3:])


def test_conv_state_continuation(rng):
    B, L, D = 2, 30, 16
    xz = i8(rng, B, L, D)
    w, bias = i8(rng, D, 4), rng.integers(-1000, 1000, size=D, dtype=np.int32)
    full, st_full = O.conv_squareplus(xz, D, w, bias)
    a, st = O.conv_squareplus(xz[:, :11], D, w, bias)
    b2, st2 = O.conv_squareplus(xz[:, 11:], D, w, bias, st)
    assert np.array_equal(np.concatenate([a, b2], 1), full) and np.array_equal(st2, st_full)


# --------------------------------------------------------------- block scan
def test_block_scan_equals_materialized_reference_dataflow(rng):
    """The fused scan equals the reference's materialized dataflow
    (mamba_integer_model.py:424-444): decay_nums and u built as [B, L, D*N]
    tensors, the elementwise scan, then y = h . C, gate, requant."""
    B, L, D, N, R = 2, 40, 16, 8, 16
    W = R + 2 * N
    xs = rng.integers(0, 128, size=(B, L, D), dtype=np.int8)
    dm = rng.integers(-20, 21, size=(B, L, D), dtype=np.int8)
    xp = i8(rng, B, L, W)
    z = i8(rng, B, L, 2 * D, lo=-128)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    yo, h = O.block_scan(xs, dm, xp, R, z, D, base, 15, 13)
    dmi = dm.astype(np.int64)
    nt = np.clip(base[None, None] + dmi[..., None], 0, 32000)                  # [B,L,D,N]
    dt = np.vectorize(O.dt_q16)(dmi)
    xd = (xs.astype(np.int64) * dt + 512) >> 10
    Bm, Cm = xp[..., R:R + N].astype(np.int64), xp[..., R + N:].astype(np.int64)
    u = xd[..., None] * Bm[:, :, None, :]
    hh = O.dyadic_scan_elementwise(u.reshape(B, L, D * N), nt.reshape(B, L, D * N), 15).reshape(B, L, D, N)
    y = np.clip(np.einsum("bldn,bln->bld", hh.astype(np.int64), Cm), -2**31, 2**31 - 1)
    g = np.vectorize(O.gate_q15)(z[..., D:].astype(np.int64))
    yg = (y * g) >> 15
    expect = np.clip((yg + (1 << 12)) >> 13, -127, 127)
    assert np.array_equal(yo, expect.astype(np.int8))
    assert np.array_equal(h, hh[:, -1])


# ------------------------------------------------------------------ model
def _tiny():
    from mamba_int import ModelDims, init_random_params
    return init_random_params(ModelDims(d_model=64, n_layer=2, vocab_size=100, d_state=16, dt_rank=16), 9)


def test_model_decode_equals_prefill():
    p = _tiny()
    m = O.OracleModel(p)
    ids = np.random.default_rng(1).integers(0, 100, size=(2, 12))
    full = m.forward(ids)
    lg, st = m.prefill(ids[:, :4])
    assert np.array_equal(lg, full[:, 3])
    for t in range(4, 12):
        lg, st = m.decode_step(ids[:, t], st)
        assert np.array_equal(lg, full[:, t])


def test_model_prefill_continuation():
    p = _tiny()
    m = O.OracleModel(p)
    ids = np.random.default_rng(2).integers(0, 100, size=(1, 20))
    lg_full, st_full = m.prefill(ids)
    _, st = m.prefill(ids[:, :9])
    lg, st2 = m.prefill(ids[:, 9:], st)
    assert np.array_equal(lg, lg_full)
    for a, b in zip(st2, st_full):
        assert np.array_equal(a.h, b.h) and np.array_equal(a.conv, b.conv)


# -------------------------------------------------------------- mutations
MUTANT_PINS = {
    1: test_scan_impulse_floor_semantics,
    2: test_scan_closed_form_zero_decay,
    3: test_scan_y_saturates_once,
    4: test_bitlinear_equals_reference_f_linear,
    5: test_norm_table_and_rounding,
    6: test_bitlinear_equals_reference_f_linear,
    7: test_scan_f32_truncates_toward_zero,
    8: test_scan_f32_truncates_toward_zero,
    9: test_scan_f32_negative_impulse_floors,
}


@pytest.mark.parametrize("mutation", sorted(MUTANT_PINS))
def test_mutations_are_caught(mutation):
    """A mistake planted in the oracle (on the CPU) makes its pin fail."""
    fn = MUTANT_PINS[mutation]
    O.set_mutation(mutation)
    try:
        with pytest.raises(AssertionError):
            if fn in (test_scan_closed_form_zero_decay, test_bitlinear_equals_reference_f_linear,
                      test_norm_table_and_rounding):
                fn(np.random.default_rng(5))
            else:
                fn()
    finally:
        O.set_mutation(0)
