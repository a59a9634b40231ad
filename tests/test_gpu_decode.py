"""GPU parity of the fused decode stages against the unfused oracle ops."""
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


def _resid(rng, m, d):
    r = rng.integers(-(2**23) + 1, 2**23, size=(m, d), dtype=np.int32)
    r[0] >>= 10
    return r


@pytest.mark.parametrize("m,n,k", [(1, 80, 64), (8, 3072, 768), (16, 300, 256), (5, 32000, 768), (8, 64, 3072),
                                   (64, 300, 256), (40, 80, 768), (33, 32000, 128)])
def test_norm_bitlinear(cuda, m, n, k):
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m + n + k)
    r = _resid(rng, m, k)
    g = rng.integers(100, 400, size=k, dtype=np.int16)
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    a = O.bitshift_norm(r, g)
    got = H(ops.norm_bitlinear(T(r), T(g), T(wp), ops.OUT_INT32, n))
    assert np.array_equal(got, O.bitlinear(a, wp, O.OUT_INT32))
    got8 = H(ops.norm_bitlinear(T(r), T(g), T(wp), ops.OUT_INT8, n, shift=4))
    assert np.array_equal(got8, O.bitlinear(a, wp, O.OUT_INT8, 4))


@pytest.mark.parametrize("m,d,D", [(8, 768, 1536), (1, 128, 256), (16, 256, 512), (64, 256, 512), (23, 128, 256)])
def test_norm_in_proj_conv(cuda, m, d, D):
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * d + D)
    r = _resid(rng, m, d)
    g = np.full(d, 256, np.int16)
    wp = pack_ternary(rng.integers(-1, 2, size=(2 * D, d), dtype=np.int8))
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    xz_ref = O.bitlinear(O.bitshift_norm(r, g), wp, O.OUT_INT8, 4)
    xs_ref, st_ref = O.conv_squareplus(xz_ref.reshape(m, 1, 2 * D), D, cw, cb, st)
    stg = T(st)
    xs = torch.zeros((m, D), dtype=torch.int8, device="cuda")
    xz = torch.zeros((m, 2 * D), dtype=torch.int8, device="cuda")
    ops.norm_in_proj_conv(T(r), T(g), T(wp), 4, T(cw), T(cb), stg, xs, xz)
    assert np.array_equal(H(xs), xs_ref[:, 0])
    assert np.array_equal(H(stg), st_ref)
    assert np.array_equal(H(xz)[:, D:], xz_ref[:, D:])


@pytest.mark.parametrize("m,D,N,R", [(8, 1536, 16, 48), (1, 256, 16, 16), (16, 512, 32, 32), (3, 100, 8, 16)])
def test_dt_scan_step(cuda, m, D, N, R):
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m + D + N + R)
    W = (R + 2 * N + 15) // 16 * 16
    xp = i8(rng, m, W)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    xs = rng.integers(0, 128, size=(m, D), dtype=np.int8)
    z = i8(rng, m, 2 * D, lo=-128)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**22), 2**22, size=(m, D, N), dtype=np.int32)
    dm = O.bitlinear(np.ascontiguousarray(xp[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs.reshape(m, 1, D), dm.reshape(m, 1, D), xp.reshape(m, 1, W), R,
                                 z.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.dt_scan_step(T(xp), R, T(wdt), 2, T(xs), T(z), D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("m,D,R", [(63, 4160, 128), (64, 4096, 224), (40, 4160, 48), (30, 4096, 96),
                                   (1, 65536, 16), (33, 2048, 128), (20, 1024, 64)])
def test_quad_split_scan_step(cuda, m, D, R):
    """The batched scan step from channel-quarter x_proj partials where the
    grid has 256 blocks of 256 channels (mi_xpart_dt_scan_step's quad-split
    kernel: one, two or four tokens per block, each lane owning one channel's
    dot, dt and gate, the quad exchanging them by DPP), over the whole int32
    state range.  Covers a last block of one token (m 63 at four per block),
    one token in a four-token block (m 1), d_inner not a multiple of 256
    (4160: waves past d_inner), dt_rank from 16 to 224, and a grid under 256
    blocks (D 1024, m 20: the two-lane-per-token kernel)."""
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * 7 + D + R)
    N = 16
    W = R + 2 * N
    xs = i8(rng, m, D)
    z = i8(rng, m, 2 * D, lo=-128)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int64)
    base[::7, 3] = -50
    base[::11, 5] = 40000
    base[0, :4] = [2**31 - 1, 2**31 - 10, -2**31, -2**31 + 5]
    base = base.astype(np.int32)
    h0 = rng.integers(-2**31, 2**31, size=(m, D, N), dtype=np.int64).astype(np.int32)
    h0[:, ::5, 0] = 2**31 - 1
    h0[:, ::9, 1] = -2**31
    xq = rng.integers(-3000, 3000, size=(m, 4, W), dtype=np.int32)
    xp = np.clip((xq.sum(1) + 16) >> 5, -127, 127).astype(np.int8)
    dm = O.bitlinear(np.ascontiguousarray(xp[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs.reshape(m, 1, D), dm.reshape(m, 1, D), xp.reshape(m, 1, W), R,
                                 z.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.xpart_dt_scan_step(T(xq), 5, R, T(wdt), 2, T(xs), T(z), D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("m,k", [(2, 15), (64, 15), (5, 15), (8, 12), (3, 17)])
def test_batched_scan_step_full_range(cuda, m, k):
    """The batched scan step (two tokens per block: 24-bit multiplies at decay
    shift 15, 64-bit arithmetic at other shifts), from int8 x_proj rows and
    from int32 x_proj partials, over the whole int32 state range: states at
    INT32_MIN / INT32_MAX and uniform over int32, decay numerators below 0 and
    above 32000 before the clamp (base values up to the int32 limits), x, B and
    C over the whole int8 range.  Decay numerators are clamped to 32000, so at
    shifts 15 and 17 every decay is below one and no state can saturate; at
    shift 12 the states grow and both saturation directions occur."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(100 * m + k)
    D, N, R = 1024, 16, 48
    W = R + 2 * N
    xs = i8(rng, m, D)
    z = i8(rng, m, 2 * D, lo=-128)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int64)
    base[::7, 3] = -50
    base[::11, 5] = 40000
    base[0, :4] = [2**31 - 1, 2**31 - 10, -2**31, -2**31 + 5]
    base = base.astype(np.int32)
    h0 = rng.integers(-2**31, 2**31, size=(m, D, N), dtype=np.int64).astype(np.int32)
    h0[:, ::5, 0] = 2**31 - 1
    h0[:, ::9, 1] = -2**31
    # x_proj as four int32 partials per token; the int8 rows are their requantised sum
    xq = rng.integers(-3000, 3000, size=(m, 4, W), dtype=np.int32)
    xp = np.clip((xq.sum(1) + 16) >> 5, -127, 127).astype(np.int8)
    dm = O.bitlinear(np.ascontiguousarray(xp[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs.reshape(m, 1, D), dm.reshape(m, 1, D), xp.reshape(m, 1, W), R,
                                 z.reshape(m, 1, 2 * D), D, base, k, 13, h_state=h0)
    if k < 15:
        assert (h_ref == 2**31 - 1).any() and (h_ref == -2**31).any()
    for form in ("rows", "partials"):
        hg = T(h0)
        yo = T(np.zeros((m, D), np.int8))
        if form == "rows":
            ops.dt_scan_step(T(xp), R, T(wdt), 2, T(xs), T(z), D, T(base), k, 13, hg, yo)
        else:
            ops.xpart_dt_scan_step(T(xq), 5, R, T(wdt), 2, T(xs), T(z), D, T(base), k, 13, hg, yo)
        assert np.array_equal(H(yo), yo_ref[:, 0]), form
        assert np.array_equal(H(hg), h_ref), form


def test_row_stats_paths(cuda):
    """Embed row statistics, the RESIDUAL epilogue's atomics (GEMV and GEMM) and
    the stats-driven norms equal the reducing norm."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(17)
    V, d, D = 300, 256, 512
    emb = i8(rng, V, d)
    for T_ in (8, 300):
        ids = rng.integers(0, V, size=T_).astype(np.int64)
        stats = torch.full((3, T_, 2), 7, dtype=torch.int64, device="cuda")
        r = ops.embed(T(ids), T(emb), row_stats=stats)
        r0 = H(r).astype(np.int64)
        assert np.array_equal(H(stats[0]), np.stack([r0.sum(1), (r0 * r0).sum(1)], 1))
        assert not H(stats[1:]).any()
        a = i8(rng, T_, D)
        wp = pack_ternary(rng.integers(-1, 2, size=(d, D), dtype=np.int8))
        ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, d, out=r, res_mult=4719, res_shift=16, row_stats=stats[1])
        r1 = H(r).astype(np.int64)
        assert np.array_equal(r1, O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0.astype(np.int32), res_mult=4719,
                                              res_shift=16))
        assert np.array_equal(H(stats[1]), np.stack([r1.sum(1), (r1 * r1).sum(1)], 1))
        g = rng.integers(100, 400, size=d, dtype=np.int16)
        ref = O.bitshift_norm(r1.astype(np.int32), g)
        assert np.array_equal(H(ops.bitshift_norm(r, T(g), row_stats=stats[1])), ref)
        assert np.array_equal(H(ops.bitshift_norm(r, T(g))), ref)
        if T_ <= 16:
            wh = pack_ternary(rng.integers(-1, 2, size=(40, d), dtype=np.int8))
            got = H(ops.norm_bitlinear(r, T(g), T(wh), ops.OUT_INT32, 40, row_stats=stats[1]))
            assert np.array_equal(got, O.bitlinear(ref, wh, O.OUT_INT32))


@pytest.mark.parametrize("m,D,N,R", [(8, 1536, 16, 48), (1, 256, 16, 16), (16, 512, 32, 32), (3, 96, 8, 16),
                                     (8, 4096, 16, 128), (2, 160, 64, 112), (4, 2048, 64, 64)])
def test_xproj_dt_scan_step(cuda, m, D, N, R):
    """x_proj fused in front of the scan step equals x_proj GEMV + unfused ops."""
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * 7 + D + N + R)
    NX = R + 2 * N
    xs = rng.integers(0, 128, size=(m, D), dtype=np.int8)
    wx = pack_ternary(rng.integers(-1, 2, size=(NX, D), dtype=np.int8))
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    z = i8(rng, m, 2 * D, lo=-128)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**22), 2**22, size=(m, D, N), dtype=np.int32)
    xp = O.bitlinear(xs, wx, O.OUT_INT8, 5)
    dm = O.bitlinear(np.ascontiguousarray(xp[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs.reshape(m, 1, D), dm.reshape(m, 1, D), xp.reshape(m, 1, NX), R,
                                 z.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.xproj_dt_scan_step(T(xs), T(wx), 5, R, T(wdt), 2, T(z), D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("m,d,D,N,R,stats", [(8, 768, 1536, 16, 48, True), (1, 128, 256, 16, 16, False),
                                             (16, 256, 512, 32, 32, True), (3, 64, 96, 8, 16, True),
                                             (5, 512, 1024, 64, 128, False), (64, 768, 1536, 16, 48, True),
                                             (40, 256, 512, 32, 32, False)])
def test_xpart_decode_chain(cuda, m, d, D, N, R, stats):
    """norm + in_proj + conv with x_proj partials, then the scan step from those
    partials, equals the unfused oracle chain (norm, in_proj, conv, x_proj,
    dt_proj, block scan)."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * d + D + N + R)
    NX = R + 2 * N
    r = _resid(rng, m, d)
    g = rng.integers(100, 400, size=d, dtype=np.int16)
    wp = pack_ternary(rng.integers(-1, 2, size=(2 * D, d), dtype=np.int8))
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    wx_t = rng.integers(-1, 2, size=(NX, D), dtype=np.int8)
    wx = pack_ternary(wx_t)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**22), 2**22, size=(m, D, N), dtype=np.int32)
    # oracle chain
    xz_ref = O.bitlinear(O.bitshift_norm(r, g), wp, O.OUT_INT8, 4)
    xs_ref, st_ref = O.conv_squareplus(xz_ref.reshape(m, 1, 2 * D), D, cw, cb, st)
    xs_ref = xs_ref[:, 0]
    part_ref = np.einsum("nbc,ibc->ibn", wx_t.reshape(NX, D // 16, 16).astype(np.int64),
                         xs_ref.reshape(m, D // 16, 16).astype(np.int64))
    xp = O.bitlinear(xs_ref, wx, O.OUT_INT8, 5)
    dm = O.bitlinear(np.ascontiguousarray(xp[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs_ref.reshape(m, 1, D), dm.reshape(m, 1, D), xp.reshape(m, 1, NX), R,
                                 xz_ref.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    # device chain
    rs = None
    if stats:
        r64 = r.astype(np.int64)
        rs = T(np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    stg = T(st)
    xs = torch.zeros((m, D), dtype=torch.int8, device="cuda")
    xz = torch.zeros((m, 2 * D), dtype=torch.int8, device="cuda")
    xpart = torch.full((m, D // 16, NX), 7, dtype=torch.int32, device="cuda")
    ops.norm_in_proj_conv(T(r), T(g), T(wp), 4, T(cw), T(cb), stg, xs, xz, row_stats=rs, w_x=T(wx), xpart=xpart)
    assert np.array_equal(H(xs), xs_ref)
    assert np.array_equal(H(stg), st_ref)
    assert np.array_equal(H(xz)[:, D:], xz_ref[:, D:])
    assert np.array_equal(H(xpart), part_ref)
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.xpart_dt_scan_step(xpart, 5, R, T(wdt), 2, xs, xz, D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("T_,d,P", [(64, 2048, 128), (8, 768, 48), (3, 1100, 7), (5, 4096, 1), (2, 256, 300)])
@pytest.mark.parametrize("v2", [False, True])
def test_norm_from_stats_parts(cuda, T_, d, P, v2):
    """BitShiftNorm (both tables) from per-block row-statistics partials
    (mi_bitshift_norm_parts) equals the reducing oracle norm; the partials are an
    exact random split of each row's (sum, sum of squares), as many as 300 per
    row, over widths that end inside a 1024-channel block."""
    from mamba_int import ops
    rng = np.random.default_rng(T_ * d + P + v2)
    r = _resid(rng, T_, d) >> int(rng.integers(0, 12))
    g = rng.integers(-400, 400, size=d, dtype=np.int16)
    r64 = r.astype(np.int64)
    full = np.stack([r64.sum(1), (r64 * r64).sum(1)], 1)
    parts = rng.integers(-(2**40), 2**40, size=(T_, P, 2), dtype=np.int64)
    parts[:, -1, :] = full - parts[:, :-1, :].sum(1)
    ref = O.bitshift_norm_v2(r, g) if v2 else O.bitshift_norm(r, g)
    assert np.array_equal(H(ops.bitshift_norm(T(r), T(g), row_stats=T(parts), v2=v2)), ref)


@pytest.mark.parametrize("m,D,N,R", [(64, 4096, 16, 128), (37, 1024, 16, 48), (5, 256, 8, 16), (20, 768, 10, 16),
                                     (1, 8192, 64, 128), (3, 4352, 16, 32)])
def test_conv_step_xproj_chain(cuda, m, D, N, R):
    """The batched decode's conv step + x_proj (mi_conv_step_xproj, one block per
    token), then the scan step, equals the unfused oracle chain (conv + squareplus,
    x_proj, dt_proj, block scan); the conv state shifts in place.  Covers more
    256-channel slices than waves (D 8192, 4352), x_proj rows not a multiple of 16
    and a padded xp row."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m + D + N + R)
    NX = R + 2 * N
    xz = i8(rng, m, 2 * D, lo=-128)
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    wx = pack_ternary(rng.integers(-1, 2, size=(NX, D), dtype=np.int8))
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**22), 2**22, size=(m, D, N), dtype=np.int32)
    xs_ref, st_ref = O.conv_squareplus(xz.reshape(m, 1, 2 * D), D, cw, cb, st)
    xs_ref = xs_ref[:, 0]
    xp_ref = O.bitlinear(xs_ref, wx, O.OUT_INT8, 5)
    dm = O.bitlinear(np.ascontiguousarray(xp_ref[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs_ref.reshape(m, 1, D), dm.reshape(m, 1, D), xp_ref.reshape(m, 1, NX), R,
                                 xz.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    stg = T(st)
    xzg = T(xz)
    xs = torch.full((m, D), 5, dtype=torch.int8, device="cuda")
    W = (NX + 15) // 16 * 16
    xp = torch.full((m, W), 9, dtype=torch.int8, device="cuda")
    ops.conv_step_xproj(xzg, D, T(cw), T(cb), stg, T(wx), 5, NX, xs=xs, xp=xp)
    assert np.array_equal(H(xs), xs_ref)
    assert np.array_equal(H(stg), st_ref)
    assert np.array_equal(H(xp)[:, :NX], xp_ref)
    assert (H(xp)[:, NX:] == 9).all()
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.dt_scan_step(xp, R, T(wdt), 2, xs, xzg, D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("m,D,N,R", [(64, 4096, 16, 128), (2, 1024, 16, 48), (5, 2048, 8, 16), (3, 8192, 16, 128),
                                     (1, 1024, 16, 32), (9, 3072, 16, 64), (7, 1024, 10, 48), (33, 2048, 16, 128)])
def test_conv_step_xpart_chain(cuda, m, D, N, R):
    """The batched decode's conv step with x_proj left as int32 sums over four
    channel quarters (mi_conv_step_xpart, four blocks per token), then the scan
    step from those sums (mi_xpart_dt_scan_step, nblk 4), equals the unfused
    oracle chain.  Covers quarters of one to eight 256-channel slices (fewer
    slices than waves at D 1024 and 3072, two conv passes at D 8192), x_proj
    rows not a multiple of 16, odd batches, one token, and nstate other than 16."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(7 * m + D + N + R)
    NX = R + 2 * N
    xz = i8(rng, m, 2 * D, lo=-128)
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    wx_t = rng.integers(-1, 2, size=(NX, D), dtype=np.int8)
    wx = pack_ternary(wx_t)
    wdt = pack_ternary(rng.integers(-1, 2, size=(D, R), dtype=np.int8))
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    h0 = rng.integers(-(2**22), 2**22, size=(m, D, N), dtype=np.int32)
    xs_ref, st_ref = O.conv_squareplus(xz.reshape(m, 1, 2 * D), D, cw, cb, st)
    xs_ref = xs_ref[:, 0]
    part_ref = np.einsum("nqc,iqc->iqn", wx_t.reshape(NX, 4, D // 4).astype(np.int64),
                         xs_ref.reshape(m, 4, D // 4).astype(np.int64))
    xp_ref = O.bitlinear(xs_ref, wx, O.OUT_INT8, 5)
    dm = O.bitlinear(np.ascontiguousarray(xp_ref[:, :R]), wdt, O.OUT_DECAY_MOD, 2)
    yo_ref, h_ref = O.block_scan(xs_ref.reshape(m, 1, D), dm.reshape(m, 1, D), xp_ref.reshape(m, 1, NX), R,
                                 xz.reshape(m, 1, 2 * D), D, base, 15, 13, h_state=h0)
    stg = T(st)
    xzg = T(xz)
    xs = torch.full((m, D), 5, dtype=torch.int8, device="cuda")
    xq = torch.full((m, 4, NX), 7, dtype=torch.int32, device="cuda")
    ops.conv_step_xpart(xzg, D, T(cw), T(cb), stg, T(wx), NX, xs=xs, xpart=xq)
    assert np.array_equal(H(xs), xs_ref)
    assert np.array_equal(H(stg), st_ref)
    assert np.array_equal(H(xq), part_ref)
    hg = T(h0)
    yo = T(np.zeros((m, D), np.int8))
    ops.xpart_dt_scan_step(xq, 5, R, T(wdt), 2, xs, xzg, D, T(base), 15, 13, hg, yo)
    assert np.array_equal(H(yo), yo_ref[:, 0])
    assert np.array_equal(H(hg), h_ref)


@pytest.mark.parametrize("m,n,k", [(8, 768, 1536), (1, 768, 1536), (16, 100, 512), (3, 2048, 4096), (5, 20, 256),
                                   (16, 64, 256 * 13), (4, 96, 1600)])
def test_decode_residual_gemv(cuda, m, n, k):
    """The decode out_proj (RESIDUAL, m <= 16, K a multiple of 64): residual
    update and the atomically added row statistics of the new rows."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * n + k)
    a = i8(rng, m, k)
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(m, n), dtype=np.int32)
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16)
    rt = T(r0)
    stats = torch.zeros((m, 2), dtype=torch.int64, device="cuda")
    ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, n, out=rt, res_mult=4719, res_shift=16, row_stats=stats)
    assert np.array_equal(H(rt), ref)
    r64 = ref.astype(np.int64)
    assert np.array_equal(H(stats), np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))


@pytest.mark.parametrize("m,n,k", [(8, 768, 1536), (1, 768, 1536), (16, 100, 512), (3, 2048, 4096), (5, 20, 320),
                                   (16, 48, 64), (4, 96, 1600), (64, 2048, 4096), (37, 768, 1536)])
def test_decode_residual_parts(cuda, m, n, k):
    """The decode out_proj with per-16-feature row-statistics partials: the
    residual update equals the oracle's and each partial is the (sum, sum of
    squares) of its block of the new rows (K any multiple of 64, so the last
    256-wide chunk may be partial; n not a multiple of 16: a short last block)."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(3 * m + n + k)
    a = i8(rng, m, k)
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(m, n), dtype=np.int32)
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16)
    rt = T(r0)
    nb = (n + 15) // 16
    parts = torch.full((m, nb, 2), 7, dtype=torch.int64, device="cuda")
    ops.bitlinear_residual_parts(T(a), T(wp), rt, 4719, 16, parts)
    assert np.array_equal(H(rt), ref)
    blk = np.zeros((m, nb * 16), np.int64)
    blk[:, :n] = ref
    blk = blk.reshape(m, nb, 16)
    exp = np.stack([blk.sum(2), (blk * blk).sum(2)], -1)
    assert np.array_equal(H(parts), exp)


@pytest.mark.parametrize("path,m,n,k", [("gemm", 300, 768, 1536), ("gemm", 130, 100, 192), ("gemv", 8, 768, 1536),
                                         ("gemv", 40, 200, 512), ("parts", 8, 768, 1536), ("parts", 37, 768, 1536),
                                         ("parts", 3, 20, 320)])
def test_residual_out_clamp_every_path(cuda, path, m, n, k):
    """The SSD block's out_proj clamp (ssd_multihead.py:589-590; res_clamp on the
    RESIDUAL accumulator) on the prefill GEMM, the decode GEMV (with row
    statistics) and the statistics-partials out_proj, with a bound that binds on a
    good share of the accumulators, against the oracle."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(5 * m + n + k)
    a = i8(rng, m, k)
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(m, n), dtype=np.int32)
    c = 400
    acc = O.bitlinear(a, wp, O.OUT_INT32)
    assert 0.05 < (np.abs(acc) > c).mean() < 0.95
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16, res_clamp=c)
    rt = T(r0)
    if path == "parts":
        parts = torch.zeros((m, (n + 15) // 16, 2), dtype=torch.int64, device="cuda")
        ops.bitlinear_residual_parts(T(a), T(wp), rt, 4719, 16, parts, res_clamp=c)
        assert np.array_equal(H(parts).sum(1)[:, 0], ref.astype(np.int64).sum(1))
    else:
        stats = torch.zeros((m, 2), dtype=torch.int64, device="cuda")
        ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, n, out=rt, res_mult=4719, res_shift=16, res_clamp=c,
                      row_stats=stats, path=path)
        r64 = ref.astype(np.int64)
        assert np.array_equal(H(stats), np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    assert np.array_equal(H(rt), ref)


def _split_stats(rng, r, P):
    """Row statistics of r as P random int64 partials [m, P, 2] that sum to them."""
    r64 = r.astype(np.int64)
    full = np.stack([r64.sum(1), (r64 * r64).sum(1)], 1)
    parts = rng.integers(-(2**40), 2**40, size=(r.shape[0], P, 2), dtype=np.int64)
    parts[:, -1] = full - parts[:, :-1].sum(1)
    return parts


@pytest.mark.parametrize("m,k,P", [(8, 768, 48), (16, 768, 48), (1, 128, 8), (3, 3072, 192), (16, 3072, 192),
                                   (2, 256, 300), (5, 64, 2), (16, 64, 1), (64, 768, 48), (29, 2048, 128)])
def test_norm_stats_partials(cuda, m, k, P):
    """The norm entries take the row statistics as stats_parts partials and sum
    them: the narrow and wide norm GEMVs, the in_proj + conv stage and the
    lm_head with keys equal the oracle's norm for any split of the sums (P
    beyond 4 loads per lane group takes the kernel's extra-load loop)."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m * k + P)
    r = _resid(rng, m, k)
    g = rng.integers(100, 400, size=k, dtype=np.int16)
    parts = T(_split_stats(rng, r, P))
    a = O.bitshift_norm(r, g)
    n = 80
    wp = pack_ternary(rng.integers(-1, 2, size=(n, k), dtype=np.int8))
    got = H(ops.norm_bitlinear(T(r), T(g), T(wp), ops.OUT_INT32, n, row_stats=parts))
    assert np.array_equal(got, O.bitlinear(a, wp, O.OUT_INT32))
    keys = torch.empty((m, (n + 63) // 64), dtype=torch.int64, device="cuda")
    logits = torch.zeros((m, n), dtype=torch.int32, device="cuda")
    ops.norm_bitlinear_argmax(T(r), T(g), T(wp), n, keys, logits=logits, row_stats=parts)
    assert np.array_equal(H(logits), O.bitlinear(a, wp, O.OUT_INT32))
    D = 64
    wi = pack_ternary(rng.integers(-1, 2, size=(2 * D, k), dtype=np.int8))
    cw = i8(rng, D, 4)
    cb = rng.integers(-600, 600, size=D, dtype=np.int32)
    st = i8(rng, m, 3, D)
    xz_ref = O.bitlinear(a, wi, O.OUT_INT8, 4)
    xs_ref, st_ref = O.conv_squareplus(xz_ref.reshape(m, 1, 2 * D), D, cw, cb, st)
    stg = T(st)
    xs = torch.zeros((m, D), dtype=torch.int8, device="cuda")
    xz = torch.zeros((m, 2 * D), dtype=torch.int8, device="cuda")
    ops.norm_in_proj_conv(T(r), T(g), T(wi), 4, T(cw), T(cb), stg, xs, xz, row_stats=parts)
    assert np.array_equal(H(xs), xs_ref[:, 0])
    assert np.array_equal(H(stg), st_ref)
    assert np.array_equal(H(xz)[:, D:], xz_ref[:, D:])


@pytest.mark.parametrize("m,n,k", [(8, 32000, 768), (1, 500, 128), (16, 1000, 256), (3, 64, 3072), (64, 500, 128),
                                   (50, 32000, 2048)])
def test_lm_head_argmax_keys(cuda, m, n, k):
    """lm_head with the fused greedy pick: logits, the picked ids (first maximal
    index: every weight row is duplicated, so every logit value occurs at least
    twice) and the embedding of the picks equal the oracle's."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(m + n + k)
    r = _resid(rng, m, k)
    g = rng.integers(100, 400, size=k, dtype=np.int16)
    half = rng.integers(-1, 2, size=((n + 1) // 2, k), dtype=np.int8)
    w = np.repeat(half, 2, axis=0)[:n]
    wp = pack_ternary(w)
    logits_ref = O.bitlinear(O.bitshift_norm(r, g), wp, O.OUT_INT32)
    ids_ref = np.argmax(logits_ref, axis=1)
    r64 = r.astype(np.int64)
    stats = T(np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    keys = torch.empty((m, (n + 63) // 64), dtype=torch.int64, device="cuda")
    logits = torch.zeros((m, n), dtype=torch.int32, device="cuda")
    ops.norm_bitlinear_argmax(T(r), T(g), T(wp), n, keys, logits=logits, row_stats=stats)
    assert np.array_equal(H(logits), logits_ref)
    assert np.array_equal(H(ops.argmax_keys(keys)), ids_ref)
    keys2 = torch.empty_like(keys)
    ops.norm_bitlinear_argmax(T(r), T(g), T(wp), n, keys2, row_stats=stats)  # logits not stored
    assert np.array_equal(H(keys2), H(keys))
    # embedding of the picks, with the row statistics of layer 0 and zeroed later layers
    V, d = n, 64
    emb = i8(rng, V, d)
    ids = torch.full((m,), -1, dtype=torch.int64, device="cuda")
    rr = torch.empty((m, d), dtype=torch.int32, device="cuda")
    st = torch.full((3, m, 2), 5, dtype=torch.int64, device="cuda")
    ops.embed_argmax(keys, ids, T(emb), rr, st)
    assert np.array_equal(H(ids), ids_ref)
    er = O.embed(ids_ref, emb).astype(np.int64)
    assert np.array_equal(H(rr), er)
    assert np.array_equal(H(st)[0], np.stack([er.sum(1), (er * er).sum(1)], 1))
    assert not H(st)[1:].any()
