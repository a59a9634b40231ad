"""Pins of the multi-head SSD block rules (spec section 7) in the oracle, on the
CPU: the BitShiftNormV2 threshold cascade on exact rational variances, the
unit-vector rule against its closed form, the decay table against an
independent float evaluation, and the scan against the reference's chunked
matmul form (``ssd_multihead_forward``) where that form is exact, plus closed
forms for memoryless and reset decays and the model's decode == prefill."""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
from mamba_int import ModelDims, init_random_params, ssd_decay_table


def _ref_table_k_v2(var: Fraction) -> int:
    """The cascade of BitShiftNormV2._find_power_of_2_scale (ssd_multihead.py:
    613-629) on an exact rational var (its eps dropped), as k of scale 2^-k."""
    scale = Fraction(1)
    for j, th in enumerate((4, 16, 64, 256, 1024, 4096), start=1):
        if var >= th:
            scale = Fraction(1, 2**j)
    if var < 1:
        scale = Fraction(1)
    if var < Fraction(1, 4):
        scale = Fraction(2)
    if var < Fraction(1, 16):
        scale = Fraction(4)
    return -int(math.log2(scale))


def test_norm_v2_table(rng):
    d = 48
    rows = [rng.integers(-2**23 + 1, 2**23, size=d), rng.integers(-5, 6, size=d), np.zeros(d, np.int64),
            rng.integers(-300, 300, size=d)]
    for j in (1, 2, 4, 6, 7, -1, -2, -3):
        target = d * 4 ** (j + 8) if j > 0 else d * 4 ** (8 + j)
        v = math.isqrt(target // d)
        row = np.zeros(d, np.int64)
        row[: d // 2] = v
        row[d // 2:] = -v
        rows.append(row)
        rows.append(row + np.where(np.arange(d) == 0, 1, 0))
    r = np.array(rows, np.int32)
    g = rng.integers(-400, 400, size=d, dtype=np.int16)
    got = O.bitshift_norm_v2(r, g)
    for t in range(r.shape[0]):
        row = [int(v) for v in r[t]]
        mu = sum(row) // d
        xs = [v - mu for v in row]
        sh = 12 + _ref_table_k_v2(Fraction(sum(v * v for v in xs), d * 2**16))
        want = [max(-127, min(127, (x * int(gi) + (1 << (sh - 1))) >> sh)) for x, gi in zip(xs, g)]
        assert got[t].tolist() == want, t
    # the V2 table differs from the V1 one above var 4096 and below 1/16
    big = np.full((1, d), 2**20, np.int32)
    big[0, ::2] = -2**20
    assert not np.array_equal(O.bitshift_norm_v2(big, g), O.bitshift_norm(big, g))


def test_unit_q7_closed_forms(rng):
    assert O.unit_q7(np.array([3, 4] + [0] * 14)).tolist()[:3] == [77, 102, 0]   # 3/5, 4/5 of 128
    assert not O.unit_q7(np.zeros(16)).any()
    for v in (1, -1, 100, -127):
        e = np.zeros(32, np.int8)
        e[5] = v
        assert O.unit_q7(e)[5] == (127 if v > 0 else -127)   # 128 saturates
    for n in (16, 32, 64):
        for _ in range(200):
            v = rng.integers(-127, 128, size=n)
            q = O.unit_q7(v).astype(np.float64)
            f = 128.0 * v / math.sqrt(float((v.astype(np.int64) ** 2).sum()))
            assert np.all(np.abs(q - np.clip(f, -127, 127)) <= 1.0 + 1e-9)


def test_decay_table_against_float():
    a_log = np.array([-5.0, -2.3, -0.693, -0.2, -0.01, 0.3])
    tab = ssd_decay_table(a_log)
    assert tab.shape == (6, 255) and tab.dtype == np.int32
    for h, a in enumerate(a_log):
        a = min(-0.01, max(-2.3, a))
        for q in range(-127, 128):
            dt = max(-10.0, min(10.0, q / 16.0))
            sp = min(10.0, max(0.01, math.log1p(math.exp(dt))))
            A = min(-0.001, max(-20.0, a * sp))
            assert tab[h, q + 127] == round(math.exp(A) * 32768.0), (h, q)
    assert np.array_equal(tab[0], tab[1]) and np.array_equal(tab[4], tab[5])   # A_log clamp to [-2.3, -0.01]
    assert np.all(np.diff(tab, axis=1) <= 0)                                  # larger dt, faster decay
    assert tab.min() >= 0 and tab.max() <= 32767


def _scan_inputs(rng, B, L, H, P, N, dt=None):
    D = H * P
    W = -(-(2 * H * N + H) // 16) * 16
    xs = rng.integers(-127, 128, size=(B, L, D)).astype(np.int8)
    xp = rng.integers(-127, 128, size=(B, L, W)).astype(np.int8)
    if dt is not None:
        xp[..., 2 * H * N:2 * H * N + H] = dt
    z = rng.integers(-127, 128, size=(B, L, 2 * D)).astype(np.int8)
    return xs, xp, z


def _unit_bc(xp, H, N):
    B, L, _ = xp.shape
    bq = np.zeros((B, L, H, N), np.int64)
    cq = np.zeros((B, L, H, N), np.int64)
    for b in range(B):
        for t in range(L):
            for h in range(H):
                bq[b, t, h] = O.unit_q7(xp[b, t, h * N:(h + 1) * N])
                cq[b, t, h] = O.unit_q7(xp[b, t, H * N + h * N:H * N + (h + 1) * N])
    return bq, cq


def _finish(y, z, D, s_y):
    """Rules 7.7-7.8 on exact y [B,L,D] (int64): clamp, gate by z[..., D:], requant."""
    y = np.clip(np.clip(y, -2**31, 2**31 - 1), -(100 << 18), 100 << 18)
    g = np.vectorize(O.gate_q15)(z[..., D:].astype(np.int64))
    yg = (y * g) >> 15
    return np.clip((yg + (1 << (s_y - 1))) >> s_y, -127, 127).astype(np.int8)


def _ssd_chunked_decay_one(X, Bq, Cq, cs):
    """ssd_multihead_forward (ssd_multihead.py:92-244) with exp(A) = 1: L is the
    causal ones matrix, Y_intra = (L * CB) @ X per chunk, carry = carry +
    h_chunk_final, Y_inter = C @ h_inter.  X [B,L,H,P], Bq/Cq [B,L,H,N]; exact in
    int64."""
    B, L, H, P = X.shape
    N = Bq.shape[-1]
    Y = np.zeros((B, L, H, P), np.int64)
    carry = np.zeros((B, H, N, P), np.int64)
    for c0 in range(0, L, cs):
        x, bb, cc = X[:, c0:c0 + cs], Bq[:, c0:c0 + cs], Cq[:, c0:c0 + cs]
        n = x.shape[1]
        Lm = np.tril(np.ones((n, n), np.int64))
        CB = np.einsum("bihs,bjhs->bhij", cc, bb)
        Y[:, c0:c0 + n] += np.einsum("bhij,bjhp->bihp", Lm[None, None] * CB, x)
        Y[:, c0:c0 + n] += np.einsum("bihs,bhsp->bihp", cc, carry)
        carry = carry + np.einsum("bjhs,bjhp->bhsp", bb, x)
    return Y


@pytest.mark.parametrize("B,L,H,P,N", [(2, 11, 2, 16, 16), (1, 9, 3, 16, 32)])
def test_scan_matches_reference_chunked_form_at_unit_decay(rng, B, L, H, P, N):
    """Decay 2^15 (exp(A) = 1): the floor is exact, so the sequential oracle
    equals the reference's chunked matmul algorithm on the same unit B, C."""
    xs, xp, z = _scan_inputs(rng, B, L, H, P, N)
    D = H * P
    xs //= 8      # keep y inside the +-100 clamp for most entries, and on it for some
    tab = np.full((H, 255), 32768, np.int32)
    yo, h = O.ssd_v2_scan(xs, xp, z, D, tab, 11, H, N)
    bq, cq = _unit_bc(xp, H, N)
    Y = _ssd_chunked_decay_one(xs.reshape(B, L, H, P).astype(np.int64), bq, cq, cs=4)
    assert np.array_equal(yo, _finish(Y.reshape(B, L, D), z, D, 11))
    # final state = sum over time of B (x) x, laid out [B, H, P, N]
    hs = np.einsum("bths,bthp->bhps", bq, xs.reshape(B, L, H, P).astype(np.int64))
    assert np.array_equal(h.reshape(B, H, P, N), hs)


def test_scan_memoryless_and_reset_decays(rng):
    """tab = 0 forgets the state every step (h = B x); a table that keeps the
    state for dt >= 0 and drops it for dt < 0 restarts the running sum at each
    negative dt: closed forms that pin the dt column and the head of each tab row."""
    B, L, H, P, N = 2, 13, 2, 16, 16
    D = H * P
    dt = rng.integers(-3, 3, size=(B, L, H))
    xs, xp, z = _scan_inputs(rng, B, L, H, P, N, dt=dt)
    xs //= 16
    bq, cq = _unit_bc(xp, H, N)
    X = xs.reshape(B, L, H, P).astype(np.int64)
    tab = np.zeros((H, 255), np.int32)
    tab[1, 127:] = 32768          # head 1 keeps the state when dt >= 0; head 0 never
    yo, _ = O.ssd_v2_scan(xs, xp, z, D, tab, 10, H, N)
    Y = np.zeros((B, L, H, P), np.int64)
    for b in range(B):
        for hd in range(H):
            hstate = np.zeros((P, N), np.int64)
            for t in range(L):
                keep = hd == 1 and dt[b, t, hd] >= 0
                hstate = (hstate if keep else 0) + np.outer(X[b, t, hd], bq[b, t, hd])
                Y[b, t, hd] = hstate @ cq[b, t, hd]
    assert np.array_equal(yo, _finish(Y.reshape(B, L, D), z, D, 10))


def test_scan_state_handoff(rng):
    B, L, H, P, N = 2, 12, 2, 16, 32
    xs, xp, z = _scan_inputs(rng, B, L, H, P, N)
    tab = ssd_decay_table(rng.uniform(-2.3, -0.01, size=H))
    D = H * P
    full, hf = O.ssd_v2_scan(xs, xp, z, D, tab, 14, H, N)
    a, ha = O.ssd_v2_scan(xs[:, :5], xp[:, :5], z[:, :5], D, tab, 14, H, N)
    b, hb = O.ssd_v2_scan(xs[:, 5:], xp[:, 5:], z[:, 5:], D, tab, 14, H, N, h_state=ha)
    assert np.array_equal(np.concatenate([a, b], 1), full) and np.array_equal(hb, hf)


def test_ssd_model_decode_equals_prefill():
    dims = ModelDims(d_model=64, n_layer=2, vocab_size=120, d_state=16, dt_rank=0, block="ssd", n_heads=2,
                     d_head=32)
    m = O.OracleModel(init_random_params(dims, 5))
    ids = np.random.default_rng(2).integers(0, 120, size=(2, 10))
    full = m.forward(ids)
    _, st = m.prefill(ids[:, :4])
    for t in range(4, 10):
        lg, st = m.decode_step(ids[:, t], st)
        assert np.array_equal(lg, full[:, t]), t
