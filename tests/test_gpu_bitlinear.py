"""GPU parity of BitLinear (MFMA GEMM and register-unpack GEMV) and the block ops."""
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


def _tern(rng, n, k):
    return rng.integers(-1, 2, size=(n, k), dtype=np.int8)


def _acc_exact(a, w):
    """int8 x ternary product via float64 BLAS (exact: |sum| < 2^53)."""
    return (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)


def test_pack_matches_host(cuda, rng):
    from mamba_int import ops, pack_ternary
    w = _tern(rng, 70, 96)
    assert np.array_equal(H(ops.pack_ternary(T(w))), pack_ternary(w))


def test_gemm_config2_int32_and_requant(cuda):
    """Config 2: M4096 K768 N3072, int8 activations, ternary weights (p=1/3 each)."""
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(2)
    M, K, N = 4096, 768, 3072
    a = i8(rng, M, K)
    w = _tern(rng, N, K)
    wp = T(pack_ternary(w))
    ref = _acc_exact(a, w)
    acc = H(ops.bitlinear(T(a), wp, ops.OUT_INT32, N, path="gemm"))
    assert np.array_equal(acc, ref)
    s = 5
    q = H(ops.bitlinear(T(a), wp, ops.OUT_INT8, N, shift=s, path="gemm"))
    assert np.array_equal(q, np.clip((ref + (1 << (s - 1))) >> s, -127, 127))
    assert np.array_equal(q[:64], O.bitlinear(a[:64], pack_ternary(w), O.OUT_INT8, s))


@pytest.mark.parametrize("M,N,K", [(1, 3072, 768), (8, 80, 1536), (8, 1536, 48), (16, 100, 64),
                                   (17, 64, 768), (33, 200, 256), (64, 2048, 1024), (64, 36, 16)])
@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_bitlinear_small_m(cuda, M, N, K, path):
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(M * 7 + N + K)
    a = i8(rng, M, K)
    w = _tern(rng, N, K)
    ref = _acc_exact(a, w)
    Np = (N + 3) // 4 * 4
    out = T(np.zeros((M, Np), np.int32))
    acc = H(ops.bitlinear(T(a), T(pack_ternary(w)), ops.OUT_INT32, N, out=out, path=path))
    assert np.array_equal(acc[:, :N], ref)


@pytest.mark.parametrize("M,N,K", [(300, 84, 48), (129, 130, 96), (1000, 3072, 768)])
def test_bitlinear_kinds(cuda, M, N, K):
    """Every output kind against the oracle, with ragged M/N and a K tail."""
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(M + N + K)
    a = i8(rng, M, K)
    wp = pack_ternary(_tern(rng, N, K))
    Np = (N + 3) // 4 * 4
    for kind, shift in ((O.OUT_INT8, 4), (O.OUT_DECAY_MOD, 7)):
        out = T(np.zeros((M, Np), np.int8))
        got = H(ops.bitlinear(T(a), T(wp), kind, N, shift=shift, out=out))[:, :N]
        assert np.array_equal(got, O.bitlinear(a, wp, kind, shift)), kind
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(M, N), dtype=np.int32)
    rp = np.zeros((M, Np), np.int32)
    rp[:, :N] = r0
    rt = T(rp)
    ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, N, out=rt, res_mult=4719, res_shift=16)
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=4719, res_shift=16)
    assert np.array_equal(H(rt)[:, :N], ref)
    xs = rng.random(M).astype(np.float32) + 0.01
    outf = T(np.zeros((M, Np), np.float32))
    got = H(ops.bitlinear(T(a), T(wp), ops.OUT_FLOAT, N, out=outf, x_scale=T(xs), w_scale=0.731))[:, :N]
    ref = O.bitlinear(a, wp, O.OUT_FLOAT, x_scale=xs, w_scale=0.731)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(200, 200, 192), (130, 36, 64), (257, 129, 320), (200, 200, 768), (130, 36, 704),
                                   (257, 129, 1536), (70, 300, 1472), (130, 36, 48), (257, 129, 80),
                                   (200, 300, 112), (300, 1536, 48), (200, 80, 1536), (130, 36, 256),
                                   (300, 160, 2048), (65, 17, 512), (1000, 150, 4096),
                                   (200, 256, 768), (257, 512, 1536), (1000, 1024, 2048)])
@pytest.mark.parametrize("pad", [0, 4, 16])
def test_gemm_tile_edges(cuda, M, N, K, pad):
    """Prefill GEMM edge tiles: a K tail of 64 past the last 128-deep stage, ragged
    M and N (the int8 tile store's 16-byte runs cut short), output row pitches that
    select the staged 16-byte store (pitch % 16 == 0) or the per-lane dword
    store, and the RESIDUAL row statistics.  K = 48, 80, 112 (weight rows of 3, 5,
    7 words) take the generic kernel, with its skipped zero halves (48: the
    dt_proj depth of the d768 model).  N <= 160 with K % 256 == 0 (x_proj) takes
    the staged GEMV kernel in 64-row groups, for int8 and int32 outputs."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(M * 3 + N + K + pad)
    a = i8(rng, M, K)
    wp = pack_ternary(_tern(rng, N, K))
    ldo = (N + 15) // 16 * 16 + pad
    for kind, shift in ((O.OUT_INT8, 3), (O.OUT_DECAY_MOD, 6)):
        out = T(np.full((M, ldo), 99, np.int8))
        got = H(ops.bitlinear(T(a), T(wp), kind, N, shift=shift, out=out, path="gemm"))
        assert np.array_equal(got[:, :N], O.bitlinear(a, wp, kind, shift)), kind
        assert (got[:, N:] == 99).all(), "stored past n"
    r0 = rng.integers(-(2**22), 2**22, size=(M, N), dtype=np.int32)
    rp = np.zeros((M, ldo), np.int32)
    rp[:, :N] = r0
    rt = T(rp)
    st = torch.zeros((M, 2), dtype=torch.int64, device="cuda")
    ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, N, out=rt, res_mult=-3001, res_shift=11, path="gemm", row_stats=st)
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=r0, res_mult=-3001, res_shift=11)
    assert np.array_equal(H(rt)[:, :N], ref)
    r64 = ref.astype(np.int64)
    assert np.array_equal(H(st), np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    acc = H(ops.bitlinear(T(a), T(wp), ops.OUT_INT32, N, out=T(np.zeros((M, ldo), np.int32)), path="gemm"))
    assert np.array_equal(acc[:, :N], O.bitlinear(a, wp, O.OUT_INT32))


@pytest.mark.parametrize("M,N,K", [(65409, 256, 128), (16385, 1024, 768), (8193, 2048, 2048)])
@pytest.mark.parametrize("pad", [0, 4])
def test_large_tile_gemm(cuda, M, N, K, pad):
    """The 256 x 128-tile kernel (N % 256 == 0, K % 128 == 0, at least 512 tiles):
    a last m-tile one row deep (rows past M clamped), one 128-deep stage, 6 and 16
    stages through the three-stage ring.  int8 requant through the staged tile
    (row pitch % 16 == 0; pad 4 takes the dword-store kernel) against the exact
    product; RESIDUAL (both pitches) with row statistics against the oracle on
    the first 256 and the last 129 rows (rows are independent)."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(M + N + K + pad)
    a = i8(rng, M, K)
    w = _tern(rng, N, K)
    wp = pack_ternary(w)
    ldo = N + pad
    s = 6
    ref = _acc_exact(a, w)
    out = T(np.full((M, ldo), 99, np.int8))
    got = H(ops.bitlinear(T(a), T(wp), ops.OUT_INT8, N, shift=s, out=out, path="gemm"))
    assert np.array_equal(got[:, :N], np.clip((ref + (1 << (s - 1))) >> s, -127, 127))
    assert (got[:, N:] == 99).all(), "stored past n"
    del ref
    r0 = rng.integers(-(2**22), 2**22, size=(M, N), dtype=np.int32)
    rp = np.zeros((M, ldo), np.int32)
    rp[:, :N] = r0
    rt = T(rp)
    st = torch.zeros((M, 2), dtype=torch.int64, device="cuda")
    ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, N, out=rt, res_mult=-3001, res_shift=11, path="gemm", row_stats=st)
    rg = H(rt)[:, :N]
    for rows in (slice(0, 256), slice(M - 129, M)):
        ref = O.bitlinear(a[rows], wp, O.OUT_RESIDUAL, residual=r0[rows], res_mult=-3001, res_shift=11)
        assert np.array_equal(rg[rows], ref)
    r64 = rg.astype(np.int64)
    assert np.array_equal(H(st), np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))


def test_squareplus_every_input(cuda):
    """Squareplus over every conv output it can see (the clamp range [-51200,
    51200] and beyond), through the conv with zero taps and the value in the
    bias: the device's exact square root against the oracle, exhaustively."""
    from mamba_int import ops
    lo, hi = -51300, 51300
    D = (hi - lo + 1 + 3) // 4 * 4
    cb = (np.arange(D) + lo).astype(np.int32)
    cw = np.zeros((D, 4), np.int8)
    xz = np.zeros((1, 1, 2 * D), np.int8)
    ref, _ = O.conv_squareplus(xz, D, cw, cb)
    got = ops.conv_squareplus(T(xz), D, T(cw), T(cb))
    assert np.array_equal(H(got), ref)


def test_act_quant_and_bitlinear_float_face(cuda):
    """Drop-in BitLinear: GPU output bit-identical to the reference's CPU formula
    (rational_bitnet.py:63-111,167-213 evaluated with torch on the CPU)."""
    import torch
    import torch.nn.functional as F
    from rational_bitnet import BitLinear
    torch.manual_seed(0)
    lin = BitLinear(768, 3072)
    x = torch.randn(64, 768)
    x[0, :4] = torch.tensor([0.5, -0.5, 1.5, 2.5]) * (x[0].abs().max() / 127)  # exact .5 ties
    with torch.no_grad():
        w = lin.weight
        s_w = torch.max(w.abs().mean(), torch.tensor(1e-6))
        wq = torch.clamp(torch.round(w / s_w), -1, 1)
        sc = torch.amax(torch.abs(x), dim=-1, keepdim=True).clamp(min=1e-8)
        xq = torch.round(x * (127 / sc)).clamp(-127, 127)
        ref = F.linear(xq, wq) * (s_w * (sc / 127))
    got = lin.cuda()(x.cuda()).cpu()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    q, s = O.act_quant_f32(x.numpy())
    from mamba_int import ops
    qg, sg = ops.act_quant(x.cuda())
    assert np.array_equal(H(qg), q) and np.array_equal(H(sg).view(np.uint32), s.view(np.uint32))
    assert np.array_equal(q, xq.numpy().astype(np.int8))


def test_norm(cuda, rng):
    from mamba_int import ops
    for T_, d in ((37, 768), (5, 2048), (3, 100), (64, 16), (9, 1536), (3, 4096), (3, 256), (6, 3072)):
        r = rng.integers(-(2**23) + 1, 2**23, size=(T_, d), dtype=np.int32)
        r[0] = 0
        r[1] = rng.integers(-3, 4, size=d)
        r[2] >>= 12
        g = rng.integers(-400, 400, size=d, dtype=np.int16)
        assert np.array_equal(H(ops.bitshift_norm(T(r), T(g))), O.bitshift_norm(r, g))


@pytest.mark.parametrize("B,L", [(2, 1), (2, 2), (1, 3), (3, 17), (2, 100)])
def test_conv_squareplus(cuda, B, L):
    from mamba_int import ops
    rng = np.random.default_rng(B * 100 + L)
    D, W = 64, 160
    xz = i8(rng, B, L, W)
    w = i8(rng, D, 4)
    bias = rng.integers(-60000, 60000, size=D, dtype=np.int32)
    st = i8(rng, B, 3, D)
    xs_ref, st_ref = O.conv_squareplus(xz, D, w, bias, st)
    stg = T(st)
    xs = ops.conv_squareplus(T(xz), D, T(w), T(bias), state_in=stg, state_out=stg)
    assert np.array_equal(H(xs), xs_ref)
    assert np.array_equal(H(stg), st_ref)
    xs0_ref, _ = O.conv_squareplus(xz, D, w, bias, None)
    assert np.array_equal(H(ops.conv_squareplus(T(xz), D, T(w), T(bias))), xs0_ref)


@pytest.mark.parametrize("B,L,D,N", [(2, 100, 64, 16), (1, 1, 32, 16), (2, 70, 48, 16), (1, 33, 32, 32), (1, 20, 16, 8)])
def test_block_scan(cuda, B, L, D, N):
    from mamba_int import ops
    rng = np.random.default_rng(B + L + D + N)
    R = 16
    W = R + 2 * N
    W = (W + 15) // 16 * 16
    xs = rng.integers(0, 128, size=(B, L, D), dtype=np.int8)
    dm = rng.integers(-20, 21, size=(B, L, D), dtype=np.int8)
    xp = i8(rng, B, L, W)
    z = i8(rng, B, L, 2 * D)
    base = rng.integers(0, 32001, size=(D, N), dtype=np.int32)
    base[0, 0] = 0
    base[-1, -1] = 32000
    h0 = rng.integers(-(2**22), 2**22, size=(B, D, N), dtype=np.int32)
    yo_ref, h_ref = O.block_scan(xs, dm, xp, R, z, D, base, 15, 14, h_state=h0)
    hg = T(h0)
    yo = ops.block_scan(T(xs), T(dm), T(xp), R, T(z), D, T(base), 15, 14, h_in=hg, h_out=hg)
    assert np.array_equal(H(yo), yo_ref)
    assert np.array_equal(H(hg), h_ref)


def test_embed_and_argmax(cuda, rng):
    import torch
    from mamba_int import ops
    emb = i8(rng, 50, 32)
    ids = rng.integers(0, 50, size=(7,)).astype(np.int64)
    assert np.array_equal(H(ops.embed(T(ids), T(emb))), O.embed(ids, emb))
    lg = rng.integers(-5, 5, size=(6, 1000), dtype=np.int32)
    lg[2, 10] = lg[2, 700] = 100  # tie: first index wins
    assert np.array_equal(H(ops.argmax(T(lg))), np.argmax(lg, axis=1))
    assert torch.equal(ops.argmax(T(lg)).cpu(), torch.argmax(torch.from_numpy(lg), dim=1))


@pytest.mark.parametrize("M,N,K", [(64, 8192, 512), (40, 4096, 256), (17, 100, 256), (64, 300, 4096), (33, 4100, 256),
                                   (64, 8192, 2048), (50, 4096, 2048), (20, 4096, 1536)])
def test_batched_decode_gemv_kinds(cuda, M, N, K):
    """The batched decode GEMV (16 < m <= 64, K a multiple of 256; 16 or 32
    features per block): every epilogue kind, and the residual's row
    statistics, against the oracle."""
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(M + N + K)
    a = i8(rng, M, K)
    w = _tern(rng, N, K)
    wp = pack_ternary(w)
    Np = (N + 3) // 4 * 4
    acc = H(ops.bitlinear(T(a), T(wp), ops.OUT_INT32, N, out=T(np.zeros((M, Np), np.int32)), path="gemv"))
    assert np.array_equal(acc[:, :N], _acc_exact(a, w))
    for kind, shift in ((O.OUT_INT8, 6), (O.OUT_DECAY_MOD, 7)):
        got = H(ops.bitlinear(T(a), T(wp), kind, N, shift=shift, out=T(np.zeros((M, Np), np.int8)), path="gemv"))
        assert np.array_equal(got[:, :N], O.bitlinear(a, wp, kind, shift)), kind
    r0 = rng.integers(-(2**23) + 1, 2**23, size=(M, Np), dtype=np.int32)
    rt = T(r0)
    stats = torch.zeros((M, 2), dtype=torch.int64, device="cuda")
    ops.bitlinear(T(a), T(wp), ops.OUT_RESIDUAL, N, out=rt, res_mult=4719, res_shift=16, row_stats=stats, path="gemv")
    ref = O.bitlinear(a, wp, O.OUT_RESIDUAL, residual=np.ascontiguousarray(r0[:, :N]), res_mult=4719, res_shift=16)
    assert np.array_equal(H(rt)[:, :N], ref)
    r64 = ref.astype(np.int64)
    assert np.array_equal(H(stats), np.stack([r64.sum(1), (r64 * r64).sum(1)], 1))
    xs = rng.random(M).astype(np.float32) + 0.01
    got = H(ops.bitlinear(T(a), T(wp), ops.OUT_FLOAT, N, out=T(np.zeros((M, Np), np.float32)), x_scale=T(xs),
                          w_scale=0.731, path="gemv"))[:, :N]
    assert np.array_equal(got.view(np.uint32), O.bitlinear(a, wp, O.OUT_FLOAT, x_scale=xs, w_scale=0.731).view(np.uint32))
