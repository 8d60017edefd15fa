"""The integer tier on the kernels that run the layer (north star: "the int32
per-block dot products must match the reference's q40.h/tq2.h"). zz_moe_dots runs a
forward on diagnostics builds of the four hot-path FFN kernels -- the matrix-core
gate/up and down kernels (v_mfma_i32_16x16x32_i8 over 1-4 token tiles, and
v_mfma_i32_4x4x4_16b_i8 with one or two token sets) and the decode GEMV kernels
(v_dot4, S <= 2, tq2 S <= 4) -- which also store every per-block int32 dot before
its fp32 scaling. Each is compared, exactly, with the dot of the reference's
integer codes (q4_0 q - 8, q40.h:179-186; q8_0 q, q40.h:374-414; tq2 c - 1,
tq2.h:134-155) against the int8 activations the kernel read: the q8_0 input of each
token, and the q8_0 hidden of each (token, slot) pair for down.

Raw forms: q4_0 enters the kernels as 16*(q - 8), so its dots are 16 times the
reference's; tq2 on the decode path is sum c*x with c in {0, 1, 2}, i.e. the
reference's dot plus the block's sum of x.
"""
import sys

import numpy as np
import pytest

import zzref as Z
import zunzuncito_amd as zz
from test_gpu_parity import _item_buckets, gpu_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def dev():
    return zz.init()


def codes(fmt, T, O, I):
    """Integer weight codes [O, I/32, 32] of a reference-layout tensor: q4_0 q - 8
    (byte j of a block: element j low nibble, j + 16 high), q8_0 q, tq2 c - 1 (byte k
    of a 64-group: elements k, k+16, k+32, k+48 at bits 0, 2, 4, 6; tq2.h:46-51)."""
    nb = I // 32
    if fmt == Z.FMT_Q40:
        b = T[:O * nb * 18].reshape(O, nb, 18)[:, :, 2:].astype(np.int32)
        return np.concatenate([b & 15, b >> 4], axis=2) - 8
    if fmt == Z.FMT_Q80:
        return T[:O * nb * 34].reshape(O, nb, 34)[:, :, 2:].view(np.int8).astype(np.int32)
    c = T[O * 4:O * 4 + O * I // 4].reshape(O, I // 64, 16).astype(np.int32)
    w = np.stack([(c >> (2 * q)) & 3 for q in range(4)], axis=2).reshape(O, I // 64, 64) - 1
    return w.reshape(O, nb, 32)


def bdots(W, x):
    """[O, nb] block dots of codes W [O, nb, 32] with int8 x [nb * 32]."""
    return np.einsum("onk,nk->on", W, x.astype(np.int32).reshape(W.shape[1], 32))


def test_codes_helper_matches_oracle_blockdots(dev):
    """The numpy decode of the reference layouts above against the oracle's pinned
    brute-force orc_blockdots, for all three formats."""
    rng = np.random.default_rng(3)
    for kind, kw in (("gemma", dict(E=2, D=512, MI=256)), ("lfm", dict(E=2, D=512, MI=256, fmts=(2, 2, 2))),
                     ("maple", dict(E=2, D=512, MI=256))):
        L = Z.make_layer(kind, seed=5, **kw)
        g, u, d = L.tensor_sizes()
        rec = L.experts[:L.esz]
        for off, fmt, (O, I) in ((0, L.fmts[0], (L.MI, L.D)), (g + u, L.fmts[2], (L.D, L.MI))):
            T = rec[off:off + Z.tensor_bytes(fmt, O, I)]
            x = rng.integers(-127, 128, I, dtype=np.int8)
            got = bdots(codes(fmt, T, O, I), x)
            for r in (0, 7, O - 1):
                row = T[O * 4 + r * (I // 4):] if fmt == Z.FMT_TQ2 else \
                    T[r * (I // 32) * (18 if fmt == Z.FMT_Q40 else 34):]
                want = np.zeros(I // 32, np.int32)
                Z.oracle().orc_blockdots(fmt, Z.ptr(np.ascontiguousarray(row)), Z.ptr(x), I, Z.ptr(want))
                assert np.array_equal(got[r], want), (kind, fmt, r)


def saturate(L):
    """Expert weights at the code extremes: every q4_0 / q8_0 row alternates blocks of
    all-minimum and all-maximum codes (q4_0 nibbles 0 and 15, q8_0 -127 and 127)."""
    g, u, d = L.tensor_sizes()
    for e in range(L.E):
        rec = L.experts[e * L.esz:(e + 1) * L.esz]
        for off, fmt, (O, I) in ((0, L.fmts[0], (L.MI, L.D)), (g, L.fmts[1], (L.MI, L.D)),
                                 (g + u, L.fmts[2], (L.D, L.MI))):
            bs = 18 if fmt == Z.FMT_Q40 else 34
            blk = rec[off:off + O * (I // 32) * bs].reshape(O, I // 32, bs)
            lo, hi = (0x00, 0xFF) if fmt == Z.FMT_Q40 else (0x81, 0x7F)
            blk[:, 0::2, 2:] = lo
            blk[:, 1::2, 2:] = hi
    return L


def check_dots(L, m, x, label):
    S, K = x.shape[0], L.K
    up, dn = m.dots(x)
    d = m.debug(S)
    eidx = np.full(S * K, -1, np.int32)
    for u_, e in enumerate(d["uniq"]):
        for n in range(d["offs"][u_], d["offs"][u_ + 1]):
            eidx[d["rows"][n] * K + d["slots"][n]] = e
    assert (eidx >= 0).all()
    g, u, dd = L.tensor_sizes()
    sizes = ((0, L.fmts[0], (L.MI, L.D)), (g, L.fmts[1], (L.MI, L.D)), (g + u, L.fmts[2], (L.D, L.MI)))
    cache = {}
    dec = S <= (4 if L.fmts[0] == Z.FMT_TQ2 else 2)

    def raw(fmt, v, x8):
        if fmt == Z.FMT_Q40:
            return 16 * v
        if fmt == Z.FMT_TQ2 and dec:                       # sum c*x = sum (c-1)*x + sum x
            return v + x8.astype(np.int32).reshape(-1, 32).sum(1)[None, :]
        return v

    for p in range(S * K):
        e, s = int(eidx[p]), p // K
        if e not in cache:
            rec = L.experts[e * L.esz:(e + 1) * L.esz]
            cache[e] = [codes(f, rec[o:o + Z.tensor_bytes(f, O, I)], O, I) for o, f, (O, I) in sizes]
        Wg, Wu, Wd = cache[e]
        xs, hs = d["xq"][s], d["hq"][p]
        for t, (W, fmt) in enumerate(((Wg, L.fmts[0]), (Wu, L.fmts[1]))):
            want = raw(fmt, bdots(W, xs), xs)
            bad = up[p, t] != want
            assert not bad.any(), (label, "up", p, t, int(bad.sum()), np.argwhere(bad)[:3])
        want = raw(L.fmts[2], bdots(Wd, hs), hs)
        bad = dn[p] != want
        assert not bad.any(), (label, "down", p, int(bad.sum()), np.argwhere(bad)[:3])
    return eidx


CASES = [
    # gemma-shaped q4_0, top-2 over 8 experts: decode (S 1, 2), items of <= 4 tokens,
    # 5-8 tokens (two token sets) and 1-4 token tiles of 16
    ("gemma", dict(E=8, K=2, D=512, MI=256), (1, 2, 3, 12, 24, 100, 160, 200), False),
    ("gemma", dict(E=8, K=2, D=512, MI=256), (1, 3, 40), True),
    # q4_0 gate/up with q8_0 down, and q8_0 throughout
    ("lfm", dict(E=8, K=2, D=1024, MI=512), (1, 2, 12, 100), False),
    ("lfm", dict(E=8, K=2, D=1024, MI=512, fmts=(2, 2, 2)), (2, 3, 40), False),
    ("lfm", dict(E=8, K=2, D=1024, MI=512, fmts=(2, 2, 2)), (1, 20), True),
    # tq2: decode up to S = 4, then the matrix cores
    ("maple", dict(E=8, K=2, D=1024, MI=512), (1, 4, 8, 60), False),
]


@pytest.mark.parametrize("kind,kw,sizes,sat", CASES)
def test_kernel_int32_dots_exact(dev, kind, kw, sizes, sat):
    L = Z.make_layer(kind, seed=13, **kw)
    if sat:
        saturate(L)
    m = gpu_layer(L)
    seen = set()
    try:
        for S in sizes:
            label = f"{kind} {kw.get('fmts', '')} S={S}{' saturated' if sat else ''}"
            say("case", label)
            x = Z.make_input(L, S, 17)
            if sat:                                   # +-1 per block: every code +-127
                x = np.where(np.arange(L.D) // 32 % 3 == 0, -1.0, 1.0).astype(np.float32)[None, :].repeat(S, 0)
                x += np.float32(0.25) * (np.arange(S, dtype=np.float32)[:, None] % 2)
            eidx = check_dots(L, m, x, label)
            dec = S <= (4 if L.fmts[0] == Z.FMT_TQ2 else 2)
            seen |= {"decode"} if dec else _item_buckets(eidx, L.E)
    finally:
        m.close()
    say("  bodies", sorted(map(str, seen)))
    if not sat and kind == "gemma":
        assert seen >= {"decode", "tiny", "two-set", 1, 2, 3, 4}, seen
