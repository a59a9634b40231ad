"""Writes the golden fixtures of tests/golden/*.npz.

The expected outputs come from this file's own pure-Python restatement of the
integer rules (Python integers, floor division, no numpy arithmetic), written
independently of the C oracle, so the committed vectors check the oracle and
the GPU path against a second implementation.  Inputs are seeded.

    python tests/golden/make_golden.py
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def sat(v, lo, hi):
    return max(lo, min(hi, v))


def rshr(v, s):
    return v if s == 0 else (v + (1 << (s - 1))) >> s


def scan(x, b, c, n, k, h0):
    B, L, D = x.shape
    N = b.shape[-1]
    y = np.zeros((B, L, D), np.int64)
    hs = h0.astype(np.int64).copy()
    for bb in range(B):
        for d in range(D):
            h = [int(v) for v in hs[bb, d]]
            for t in range(L):
                acc = 0
                for j in range(N):
                    h[j] = sat((h[j] * int(n[d, j])) // (1 << k) + int(b[bb, t, j]) * int(x[bb, t, d]), -2**31, 2**31 - 1)
                    acc += int(c[bb, t, j]) * h[j]
                y[bb, t, d] = sat(acc, -2**31, 2**31 - 1)
            hs[bb, d] = h
    return y.astype(np.int32), hs.astype(np.int32)


def ternary_acc(a, w):
    M, K = a.shape
    N = w.shape[0]
    out = np.zeros((M, N), np.int64)
    for m in range(M):
        for nn in range(N):
            out[m, nn] = sum(int(a[m, kk]) * int(w[nn, kk]) for kk in range(K))
    return out


def pack(w):
    N, K = w.shape
    out = np.zeros((N, K // 4), np.uint8)
    for nn in range(N):
        for wd in range(K // 16):
            word = 0
            for q in range(16):
                code = {0: 0, 1: 1, -1: 3}[int(w[nn, 16 * wd + q])]
                word |= code << (8 * (q % 4) + 2 * (q // 4))
            out[nn, 4 * wd:4 * wd + 4] = list(word.to_bytes(4, "little"))
    return out


def norm(r, gamma):
    T, d = r.shape
    out = np.zeros((T, d), np.int8)
    for t in range(T):
        row = [int(v) for v in r[t]]
        mu = sum(row) // d
        S = sum((v - mu) ** 2 for v in row)
        k = sum(1 for j in range(1, 9) if S >= d * 4 ** (j + 8)) - sum(1 for j in range(1, 4) if S < d * 4 ** (8 - j))
        for i in range(d):
            out[t, i] = sat(rshr((row[i] - mu) * int(gamma[i]), 12 + k), -127, 127)
    return out


def squareplus(c):
    v = sat(int(c), -51200, 51200)
    return sat(rshr(v + math.isqrt(v * v + (1 << 22)), 7), -127, 127)


def conv_sqp(x, w, bias, st):
    B, L, D = x.shape
    xs = np.zeros((B, L, D), np.int8)
    st_out = st.copy()
    for bb in range(B):
        for d in range(D):
            win = [int(v) for v in st[bb, :, d]]
            for t in range(L):
                xv = int(x[bb, t, d])
                c = int(bias[d]) + sum(int(w[d, j]) * win[j] for j in range(3)) + int(w[d, 3]) * xv
                xs[bb, t, d] = squareplus(c)
                win = win[1:] + [xv]
            st_out[bb, :, d] = win
    return xs, st_out


def dt_q16(dm):
    s = dm * 65536 + math.isqrt(dm * dm * 2**32 + 2**34)
    return sat(rshr(655 * (s >> 1), 16), 66, 6554)


def gate_q15(z):
    a = abs(z)
    q = (16384 * a) // (16 + a)
    return 16384 + (q if z >= 0 else -q)


def block_scan(xs, dm, xp, R, z, base, k, s_y, h0):
    B, L, D = xs.shape
    N = base.shape[1]
    yo = np.zeros((B, L, D), np.int8)
    hs = h0.astype(np.int64).copy()
    for bb in range(B):
        for d in range(D):
            h = [int(v) for v in hs[bb, d]]
            for t in range(L):
                dmv = sat(int(dm[bb, t, d]), -20, 20)
                xd = rshr(int(xs[bb, t, d]) * dt_q16(dmv), 10)
                acc = 0
                for j in range(N):
                    nt = sat(int(base[d, j]) + dmv, 0, 32000)
                    h[j] = sat((h[j] * nt) // (1 << k) + int(xp[bb, t, R + j]) * xd, -2**31, 2**31 - 1)
                    acc += int(xp[bb, t, R + N + j]) * h[j]
                y = sat(acc, -2**31, 2**31 - 1)
                yg = (y * gate_q15(int(z[bb, t, d]))) >> 15
                yo[bb, t, d] = sat(rshr(yg, s_y), -127, 127)
            hs[bb, d] = h
    return yo, hs.astype(np.int32)


def main():
    rng = np.random.default_rng(20261201)

    def i8(*shape, lo=-127, hi=127):
        return rng.integers(lo, hi + 1, size=shape, dtype=np.int8)

    # scan, config-1 layout (B2 L24 D8 N16), with a non-zero initial state
    x, b, c = i8(2, 24, 8), i8(2, 24, 16), i8(2, 24, 16, lo=-128)
    n = rng.integers(16384, 32768, size=(8, 16), dtype=np.int32)
    h0 = rng.integers(-2**24, 2**24, size=(2, 8, 16), dtype=np.int32)
    y, h = scan(x, b, c, n, 15, h0)
    np.savez(os.path.join(HERE, "scan_c1_small.npz"), x=x, b=b, c=c, n=n, h0=h0, y=y, h=h)

    # chunked multi-head scan (B1 L40 H2 P16 N32; per-head decay), expected from the
    # channel scan per head
    L, H, P, N = 40, 2, 16, 32
    xs4, bs4, cs4 = i8(1, L, H, P), i8(1, L, H, N), i8(1, L, H, N)
    n4 = rng.integers(24576, 32768, size=(H,), dtype=np.int32)
    y4 = np.zeros((1, L, H, P), np.int32)
    for hd in range(H):
        y4[:, :, hd], _ = scan(xs4[:, :, hd], bs4[:, :, hd], cs4[:, :, hd], np.full((P, N), n4[hd], np.int32), 15,
                               np.zeros((1, P, N), np.int32))
    np.savez(os.path.join(HERE, "ssd_small.npz"), x=xs4, b=bs4, c=cs4, n=n4, chunk=np.int32(16), y=y4)

    # BitLinear: int8 x ternary, packed bytes, int32 and requantized outputs
    a = i8(9, 48)
    w = rng.integers(-1, 2, size=(20, 48), dtype=np.int8)
    acc = ternary_acc(a, w)
    q5 = np.vectorize(lambda v: sat(rshr(int(v), 5), -127, 127))(acc).astype(np.int8)
    np.savez(os.path.join(HERE, "bitlinear_small.npz"), a=a, w=w, packed=pack(w), acc=acc.astype(np.int32), q5=q5)

    # BitShiftNorm over rows of very different scale
    r = np.concatenate([rng.integers(-2**23 + 1, 2**23, size=(3, 64)), rng.integers(-40, 40, size=(3, 64)),
                        rng.integers(-3000, 3000, size=(2, 64))]).astype(np.int32)
    g = rng.integers(64, 512, size=64, dtype=np.int16)
    np.savez(os.path.join(HERE, "norm_small.npz"), r=r, gamma=g, out=norm(r, g))

    # conv + squareplus with an initial conv state
    xc = i8(2, 7, 16)
    wc = i8(16, 4)
    bc = rng.integers(-30000, 30000, size=16, dtype=np.int32)
    st = i8(2, 3, 16)
    xsc, st_out = conv_sqp(xc, wc, bc, st)
    np.savez(os.path.join(HERE, "conv_sqp_small.npz"), x=xc, w=wc, bias=bc, state=st, xs=xsc, state_out=st_out)

    # fused model scan (B2 L12 D16 N16, R16)
    R, N = 16, 16
    xsb = rng.integers(0, 128, size=(2, 12, 16), dtype=np.int8)
    dmb = rng.integers(-20, 21, size=(2, 12, 16), dtype=np.int8)
    xpb = i8(2, 12, R + 2 * N)
    zb = i8(2, 12, 16, lo=-128)
    base = rng.integers(0, 32001, size=(16, N), dtype=np.int32)
    hb0 = rng.integers(-2**20, 2**20, size=(2, 16, N), dtype=np.int32)
    yo, hb = block_scan(xsb, dmb, xpb, R, zb, base, 15, 13, hb0)
    np.savez(os.path.join(HERE, "block_scan_small.npz"), xs=xsb, dm=dmb, xp=xpb, z=zb, base=base, h0=hb0, yo=yo, h=hb)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
