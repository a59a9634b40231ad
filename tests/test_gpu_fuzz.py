"""Seeded random-shape sweeps of the GPU entry points against the oracle:
ragged sizes inside each entry's documented limits, every output kind and
dispatch path, state in and out.  Each case prints nothing and runs in
milliseconds; the seeds make every shape reproducible."""
import numpy as np
import pytest

import oracle as O
from conftest import i8
from mamba_int import pack_ternary, ssd_decay_table

pytestmark = pytest.mark.gpu


def T(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def H(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("seed", range(12))
def test_bitlinear_random_shapes(cuda, seed):
    """Every kind on the auto, GEMM and GEMV paths (GEMV only for m <= 64)."""
    from mamba_int import ops
    rng = np.random.default_rng(1000 + seed)
    m = int(rng.choice([1, 3, 16, 17, 40, 64, 65, 130, 300]))
    n = int(rng.integers(1, 400))
    k = 16 * int(rng.integers(1, 80))
    a = i8(rng, m, k)
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    s = int(rng.integers(0, 12))
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(m, n), dtype=np.int32)
    mult, rsh = int(rng.integers(-70000, 70000)), int(rng.integers(0, 24))
    clamp = int(rng.choice([0, 0, 1, 40, 300, 2000]))         # RESIDUAL accumulator bound, 0 = none
    refs = {ops.OUT_INT32: O.bitlinear(a, wp, O.OUT_INT32),
            ops.OUT_INT8: O.bitlinear(a, wp, O.OUT_INT8, s),
            ops.OUT_DECAY_MOD: O.bitlinear(a, wp, O.OUT_DECAY_MOD, s),
            ops.OUT_RESIDUAL: O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=mult, res_shift=rsh,
                                          res_clamp=clamp)}
    import torch
    ldo = n + (-n) % 4                      # output rows: a multiple of 4 elements
    dtypes = {ops.OUT_INT32: torch.int32, ops.OUT_INT8: torch.int8, ops.OUT_DECAY_MOD: torch.int8}
    for path in ("auto", "gemm") + (("gemv",) if m <= 64 else ()):
        for kind, ref in refs.items():
            if kind == ops.OUT_RESIDUAL:
                out = T(np.pad(r0, ((0, 0), (0, ldo - n))))
                ops.bitlinear(T(a), T(wp), kind, n, out=out, res_mult=mult, res_shift=rsh, res_clamp=clamp,
                              path=path)
            else:
                out = torch.zeros((m, ldo), dtype=dtypes[kind], device="cuda")
                ops.bitlinear(T(a), T(wp), kind, n, shift=s, out=out, path=path)
            assert np.array_equal(H(out)[:, :n], ref), (path, kind, m, n, k, clamp)


@pytest.mark.parametrize("seed", range(8))
def test_block_scan_random_shapes(cuda, seed):
    """Fused model scan (dyadic block) over random batch, length, width and N,
    from a random state, against the oracle (outputs and final state)."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(2000 + seed)
    B = int(rng.integers(1, 5))
    L = int(rng.integers(1, 200))
    D = 16 * int(rng.integers(1, 24))
    N = int(rng.choice([16, 32, 64]))
    R = 16
    W = R + 2 * N
    xs = rng.integers(0, 128, size=(B, L, D)).astype(np.int8)
    dm = rng.integers(-20, 21, size=(B, L, D)).astype(np.int8)
    xp = i8(rng, B, L, W)
    z = i8(rng, B, L, 2 * D)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**24), 2**24, size=(B, D, N), dtype=np.int32)
    ref_y, ref_h = O.block_scan(xs, dm, xp, R, z, D, base, 15, 13, h_state=h0)
    h = T(h0)
    y = ops.block_scan(T(xs), T(dm), T(xp), R, T(z), D, T(base), 15, 13, h_in=h, h_out=h)
    assert np.array_equal(H(y), ref_y) and np.array_equal(H(h), ref_h), (B, L, D, N)
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", range(8))
def test_ssd_scan_random_shapes(cuda, seed):
    from mamba_int import ops
    rng = np.random.default_rng(3000 + seed)
    B = int(rng.integers(1, 4))
    L = int(rng.integers(1, 150))
    Hh = int(rng.integers(1, 6))
    P = 16 * int(rng.integers(1, 6))
    N = int(rng.choice([16, 32, 64]))
    D = Hh * P
    Wd = -(-(2 * Hh * N + Hh) // 16) * 16
    xs, xp, xz = i8(rng, B, L, D), i8(rng, B, L, Wd), i8(rng, B, L, 2 * D)
    tab = ssd_decay_table(rng.uniform(-2.3, -0.01, size=Hh))
    h0 = rng.integers(-(2**25), 2**25, size=(B, D, N), dtype=np.int32)
    s_y = int(rng.integers(8, 16))
    ref_y, ref_h = O.ssd_v2_scan(xs, xp, xz, D, tab, s_y, Hh, N, h_state=h0)
    h = T(h0)
    y = ops.ssd_block_scan(T(xs), T(xp), T(xz), D, T(tab), Hh, N, s_y, h_in=h, h_out=h)
    assert np.array_equal(H(y), ref_y) and np.array_equal(H(h), ref_h), (B, L, Hh, P, N)


@pytest.mark.parametrize("seed", range(8))
def test_norm_and_conv_random_shapes(cuda, seed):
    """Both norm tables, reducing and from row statistics; conv + squareplus
    over ragged lengths with a carried state."""
    from mamba_int import ops
    rng = np.random.default_rng(4000 + seed)
    T_ = int(rng.integers(1, 300))
    d = 4 * int(rng.integers(1, 400))
    r = rng.integers(-(2**23) + 1, 2**23, size=(T_, d), dtype=np.int32) >> int(rng.integers(0, 20))
    g = rng.integers(-500, 500, size=d, dtype=np.int16)
    r64 = r.astype(np.int64)
    st = T(np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    for v2, ref in ((False, O.bitshift_norm(r, g)), (True, O.bitshift_norm_v2(r, g))):
        assert np.array_equal(H(ops.bitshift_norm(T(r), T(g), v2=v2)), ref)
        assert np.array_equal(H(ops.bitshift_norm(T(r), T(g), row_stats=st, v2=v2)), ref)
    B, L, D = int(rng.integers(1, 4)), int(rng.integers(1, 70)), 4 * int(rng.integers(1, 100))
    xz = i8(rng, B, L, 2 * D)
    cw, cb = i8(rng, D, 4), rng.integers(-3000, 3000, size=D, dtype=np.int32)
    s0 = i8(rng, B, 3, D)
    ref_xs, ref_st = O.conv_squareplus(xz, D, cw, cb, s0)
    sg = T(s0)
    xs = ops.conv_squareplus(T(xz), D, T(cw), T(cb), state_in=sg, state_out=sg)
    assert np.array_equal(H(xs), ref_xs) and np.array_equal(H(sg), ref_st)


@pytest.mark.parametrize("seed", range(8))
def test_batched_decode_step_random_shapes(cuda, seed):
    """The batched decode's conv + x_proj stages and the scan step that
    finishes them: the int8-row form (mi_conv_step_xproj + mi_dt_scan_step)
    at any d_inner multiple of 256, and the channel-quarter form
    (mi_conv_step_xpart + mi_xpart_dt_scan_step) where d_inner is a multiple
    of 1024, both against the unfused oracle chain with state carried."""
    import torch
    from mamba_int import ops
    rng = np.random.default_rng(4000 + seed)
    m = int(rng.integers(1, 65))
    D = 256 * int(rng.integers(1, 17))
    if seed % 2 == 0:
        D = 1024 * int(rng.integers(1, 5))
    N = int(rng.choice([8, 16, 16, 32]))
    R = 16 * int(rng.integers(1, (256 - 2 * N) // 16 + 1))
    NX = R + 2 * N
    s_x, s_dt, s_y = int(rng.integers(2, 8)), int(rng.integers(0, 4)), int(rng.integers(8, 16))
    xz = i8(rng, m, 2 * D, lo=-128)
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    wx_t = rng.integers(-1, 2, size=(NX, D), dtype=np.int8)
    wx = pack_ternary(wx_t)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**24), 2**24, size=(m, D, N), dtype=np.int32)
    xs_ref, st_ref = O.conv_squareplus(xz.reshape(m, 1, 2 * D), D, cw, cb, st)
    xs_ref = xs_ref[:, 0]
    xp_ref = O.bitlinear(xs_ref, wx, O.OUT_INT8, s_x)
    dm = O.bitlinear(np.ascontiguousarray(xp_ref[:, :R]), wdt, O.OUT_DECAY_MOD, s_dt)
    yo_ref, h_ref = O.block_scan(xs_ref.reshape(m, 1, D), dm.reshape(m, 1, D), xp_ref.reshape(m, 1, NX), R,
                                 xz.reshape(m, 1, 2 * D), D, base, 15, s_y, h_state=h0)
    forms = ["row"] + (["quarters"] if D % 1024 == 0 else [])
    for form in forms:
        stg, xzg = T(st), T(xz)
        xs = torch.zeros((m, D), dtype=torch.int8, device="cuda")
        hg = T(h0)
        yo = T(np.zeros((m, D), np.int8))
        if form == "row":
            xp = torch.zeros((m, NX), dtype=torch.int8, device="cuda")
            ops.conv_step_xproj(xzg, D, T(cw), T(cb), stg, T(wx), s_x, NX, xs=xs, xp=xp)
            assert np.array_equal(H(xp), xp_ref), (form, m, D, N, R)
            ops.dt_scan_step(xp, R, T(wdt), s_dt, xs, xzg, D, T(base), 15, s_y, hg, yo)
        else:
            xq = torch.zeros((m, 4, NX), dtype=torch.int32, device="cuda")
            ops.conv_step_xpart(xzg, D, T(cw), T(cb), stg, T(wx), NX, xs=xs, xpart=xq)
            ops.xpart_dt_scan_step(xq, s_x, R, T(wdt), s_dt, xs, xzg, D, T(base), 15, s_y, hg, yo)
        assert np.array_equal(H(xs), xs_ref), (form, m, D, N, R)
        assert np.array_equal(H(stg), st_ref), (form, m, D, N, R)
        assert np.array_equal(H(yo), yo_ref[:, 0]), (form, m, D, N, R)
        assert np.array_equal(H(hg), h_ref), (form, m, D, N, R)
