"""Pins for the CPU oracle (oracle/zz_oracle.c) before anything is checked against it.

Each oracle function is checked against something that does not share its code:
the reference's own known-answer tests (tests/test_q40.c, tests/test_tq2.c),
golden vectors written by the compiled reference (tests/golden/), the compiled
reference itself where oracle/_ref exists, and closed forms (numpy's IEEE
binary16, brute-force integer dots, argsort with the lower-index tie rule).
"""
import ctypes as C
import os

import numpy as np
import pytest

import zzref as Z

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def lcg12345(n):
    """tests/test_q40.c:9-10 / test_tq2.c:16-20: rs = rs*1664525 + 1013904223."""
    out = np.empty(n, np.float32)
    rs = 12345
    for i in range(n):
        rs = (rs * 1664525 + 1013904223) & 0xffffffff
        out[i] = np.float32(np.float32(rs >> 8) / np.float32(8388608.0) - np.float32(1.0))
    return out


# ------------------------------------------------------------------- fp16 (A1)
def test_h2f_all_halves_match_numpy():
    L = Z.oracle()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.orc_h2f(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.all(np.isinf(got[np.isinf(want)]))


def test_f2h_round_half_even_matches_numpy():
    L = Z.oracle()
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32) * np.float32(s)
                         for s in (1e-9, 3e-8, 6e-5, 1e-3, 1.0, 3e4, 7e4)])
    # exact ties between two halves: RNE must pick the even one
    ties = (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)
    xs = np.concatenate([xs, ties, -ties, [0.0, -0.0, 65504.0, 65520.0, np.inf, -np.inf]]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f2h(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    # NaN: quiet, payload dropped, sign kept (q40.h:64)
    assert L.orc_f2h(float("nan")) & 0x7fff == 0x7e00


def test_fp16_roundtrip_test_q40_case1():
    """tests/test_q40.c:32-39: 200k round trips within half an fp16 ulp."""
    L = Z.oracle()
    f = lcg12345(20000) * np.float32(0.5)
    for v in f:
        g = L.orc_h2f(L.orc_f2h(float(v)))
        assert abs(v - g) <= abs(v) * (1.0 / 1024.0) + 1e-7
    assert L.orc_h2f(L.orc_f2h(0.0)) == 0.0


# ------------------------------------------------------- quantisers (A3, A7)
def test_q40_quant_contract_test_q40_case2():
    """tests/test_q40.c:41-79: max element exact, in-range error <= d/2, clamps."""
    I = 4096
    w = lcg12345(I) * np.float32(0.1)
    q = Z.quant_rows(Z.FMT_Q40, w.reshape(1, I))
    L = Z.oracle()
    wd = np.zeros(I, np.float32)
    L.orc_q40_dequant_row.argtypes = [Z.u8p, Z.f32p, C.c_int]
    L.orc_q40_dequant_row(Z.ptr(q), Z.ptr(wd), I)
    for b in range(I // 32):
        ds = np.frombuffer(q[b * 18:b * 18 + 2].tobytes(), np.float16)[0].astype(np.float32)
        d = abs(ds)
        lo, hi = (-8 * ds, 7 * ds) if ds >= 0 else (7 * ds, -8 * ds)
        blk, deq = w[b * 32:(b + 1) * 32], wd[b * 32:(b + 1) * 32]
        mx = blk[np.argmax(np.abs(blk))]
        for t, v in zip(blk, deq):
            if t == mx:
                assert abs(t - v) <= 0.01 * d + 1e-6
            if lo <= t <= hi:
                assert abs(t - v) <= 0.5 * d + 1e-6
            else:
                assert abs(v - (hi if t > hi else lo)) <= 1e-6


def _fused_differs(x, idv):
    """True where trunc(fma(x,id,8.5)) != trunc(fl(x*id)+8.5) for f32 x, id."""
    fused = np.floor(x.astype(np.float64) * np.float64(idv) + 8.5)
    unf = np.floor((x * np.float32(idv)).astype(np.float32).astype(np.float64) + 8.5)
    return fused != unf


def test_q40_quant_fused_rounding_golden():
    """The reference build fuses x*id + 8.5 (q40.h:101 under -mfma). Blocks built so
    that fused and unfused truncations disagree pin that choice: the oracle must
    reproduce the compiled reference's bytes on them."""
    L = Z.oracle()
    rng = np.random.default_rng(7)
    blocks, found = [], 0
    while found < 64:
        mx = np.float32(-rng.uniform(0.05, 0.1))
        hd = L.orc_f2h(float(mx / np.float32(-8.0)))
        d = np.float32(L.orc_h2f(hd))
        idv = np.float32(1.0) / d
        k = rng.integers(-8, 7, size=31)
        # land x*id within an ulp of k+0.5-8.5 boundaries
        x = ((k.astype(np.float64) + 0.5 - 1e-7 * rng.integers(-3, 4, size=31)) / float(idv)).astype(np.float32)
        x = np.clip(x, -abs(mx) * 0.99, abs(mx) * 0.99).astype(np.float32)
        if _fused_differs(x, idv).any():
            blocks.append(np.concatenate([[mx], x]).astype(np.float32))
            found += 1
    w = np.concatenate(blocks)
    got = Z.quant_rows(Z.FMT_Q40, w.reshape(1, -1))
    R = Z.ref_lib("kernels")
    if R is None:
        pytest.skip("oracle/_ref not built: the fused-rounding pin needs the compiled reference")
    want = np.zeros_like(got)
    R.ref_q40_quant_row(Z.ptr(w), Z.ptr(want), w.size)
    assert np.array_equal(got, want)


def test_kernel_golden_vectors():
    """Quantiser bytes, activation quantisation and all three dots against the
    compiled reference's outputs on the test_q40.c LCG stream."""
    g = np.load(os.path.join(GOLDEN, "kernels_lcg12345.npz"))
    L = Z.oracle()
    w = g["w"]
    O, I = 16, 2816
    assert np.array_equal(Z.quant_rows(Z.FMT_Q40, w.reshape(O, I)), g["q40"])
    assert np.array_equal(Z.quant_rows(Z.FMT_Q80, w.reshape(O, I)), g["q80"])
    x = g["x"]
    for t in range(4):
        xq = np.zeros(I, np.int8)
        xs = np.zeros(I // 32, np.float32)
        L.orc_quant_act(Z.ptr(np.ascontiguousarray(x[t])), Z.ptr(xq), Z.ptr(xs), I)
        assert np.array_equal(xq, g["xq"][t])
        assert np.array_equal(xs.view(np.uint32), g["xs"][t].view(np.uint32))
        for o in range(O):
            a = L.orc_q40_dot(Z.ptr(g["q40"][o * 88 * 18:]), Z.ptr(xq), Z.ptr(xs), I)
            b = L.orc_q80_dot(Z.ptr(g["q80"][o * 88 * 34:]), Z.ptr(xq), Z.ptr(xs), I)
            assert np.float32(a).view(np.uint32) == g["d40"][t, o].view(np.uint32)
            assert np.float32(b).view(np.uint32) == g["d80"][t, o].view(np.uint32)
    assert np.array_equal(Z.tq2_tensor(g["codes"], g["alpha"]), g["tq"])
    It = 2048
    q = np.zeros(It, np.int8)
    s = np.zeros(It // 32, np.float32)
    tot = L.orc_tq2_quant_act(Z.ptr(g["xt"]), Z.ptr(q), Z.ptr(s), It)
    assert np.array_equal(q, g["tq_q"]) and np.float32(tot) == g["tq_tot"]
    cb = g["tq"][16 * 4:]
    for o in range(16):
        v = L.orc_tq2_dot(Z.ptr(cb[o * 512:]), C.c_float(g["alpha"][o]), Z.ptr(q), Z.ptr(s),
                          C.c_float(tot), It)
        assert np.float32(v).view(np.uint32) == g["dtq"][o].view(np.uint32)


def test_quant_act_special_cases():
    """q40.h:124-138: zero block -> d=0, q=0; +-amax -> +-127; ties to even."""
    L = Z.oracle()
    x = np.zeros(96, np.float32)
    x[32] = 2.5
    x[33] = -2.5
    x[40] = 2.5 * 3 / 127          # exactly representable? check rint on a tie below
    d = np.float32(2.5) / np.float32(127.0)
    x[64:96] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5) * d
    x[64] = np.float32(127) * d    # block max element
    q = np.zeros(96, np.int8)
    s = np.zeros(3, np.float32)
    L.orc_quant_act(Z.ptr(x), Z.ptr(q), Z.ptr(s), 96)
    assert s[0] == 0.0 and not q[:32].any()
    assert q[32] == 127 and q[33] == -127 and s[1] == d
    idv = np.float32(1.0) / s[2]
    want = np.clip(np.rint((x[64:] * idv).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(q[64:], want)      # numpy rint is round-half-even


def test_q40_dot_vs_scalar_and_saturation_test_q40_cases3_4():
    """tests/test_q40.c:81-137: kernel vs double scalar reference within 1e-5 of
    sum|summands|; saturation known answer 128 blocks x 32 x 7 x 127 = 3,641,344."""
    L = Z.oracle()
    I = 4096
    rng = np.random.default_rng(12345)
    q = Z.quant_rows(Z.FMT_Q40, (rng.standard_normal(I) * 0.1).astype(np.float32).reshape(1, I))
    nib = np.frombuffer(q.tobytes(), np.uint8).reshape(-1, 18)
    dw = nib[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    qv = np.concatenate([(nib[:, 2:] & 15), (nib[:, 2:] >> 4)], axis=1).astype(np.int64) - 8
    worst = 0.0
    for _ in range(50):
        x = rng.standard_normal(I).astype(np.float32)
        xq = np.zeros(I, np.int8)
        xs = np.zeros(I // 32, np.float32)
        L.orc_quant_act(Z.ptr(x), Z.ptr(xq), Z.ptr(xs), I)
        blk = (qv * xq.reshape(-1, 32).astype(np.int64)).sum(1)
        summ = dw * xs.astype(np.float64) * blk
        ref = summ.sum()
        got = L.orc_q40_dot(Z.ptr(q), Z.ptr(xq), Z.ptr(xs), I)
        mag = np.abs(dw[:, None] * xs.astype(np.float64)[:, None] * qv * xq.reshape(-1, 32)).sum()
        worst = max(worst, abs(got - ref) / (mag + 1e-6))
    assert worst < 1e-5
    sat = np.zeros(I // 32 * 18, np.uint8).reshape(-1, 18)
    sat[:, 0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    sat[:, 2:] = 0xFF
    xq = np.full(I, 127, np.int8)
    xs = np.ones(I // 32, np.float32)
    got = L.orc_q40_dot(Z.ptr(sat.reshape(-1)), Z.ptr(xq), Z.ptr(xs), I)
    assert got == 3641344.0


def test_blockdots_brute_force():
    L = Z.oracle()
    rng = np.random.default_rng(3)
    I = 768
    xq = rng.integers(-127, 128, I, dtype=np.int8)
    for fmt in (Z.FMT_Q40, Z.FMT_Q80):
        row = Z.quant_rows(fmt, rng.standard_normal((1, I)).astype(np.float32))
        out = np.zeros(I // 32, np.int32)
        L.orc_blockdots(fmt, Z.ptr(row), Z.ptr(xq), I, Z.ptr(out))
        bb = 18 if fmt == Z.FMT_Q40 else 34
        blk = np.frombuffer(row.tobytes(), np.uint8).reshape(-1, bb)[:, 2:]
        if fmt == Z.FMT_Q40:
            wv = np.concatenate([blk & 15, blk >> 4], axis=1).astype(np.int64) - 8
        else:
            wv = blk.view(np.int8).astype(np.int64)
        assert np.array_equal(out, (wv * xq.reshape(-1, 32)).sum(1))
    codes = rng.integers(0, 3, size=(1, I)).astype(np.int8)
    t = Z.tq2_tensor(codes, np.ones(1, np.float32))
    out = np.zeros(I // 32, np.int32)
    L.orc_blockdots(Z.FMT_TQ2, Z.ptr(t[4:]), Z.ptr(xq), I, Z.ptr(out))
    assert np.array_equal(out, ((codes[0].astype(np.int64) - 1) * xq).reshape(-1, 32).sum(1))


# ------------------------------------------- f32-activation dots (A6, A9)
def _f32_rows(rng, fmt, O, I, specials=False):
    """Random q4_0 / q8_0 rows; with specials, some fp16 scales are NaN, +-inf, -0
    or subnormal (q40.h:46-60 decodes them all)."""
    q = Z.quant_rows(fmt, (rng.standard_normal((O, I)) * 0.05).astype(np.float32))
    if specials:
        bb = 18 if fmt == Z.FMT_Q40 else 34
        blk = q.reshape(-1, bb)
        pick = rng.choice(blk.shape[0], size=min(12, blk.shape[0]), replace=False)
        for k, b in enumerate(pick):
            h = [0x7e00, 0x7c00, 0xfc00, 0x8000, 0x0001, 0x03ff][k % 6]
            blk[b, 0], blk[b, 1] = h & 255, h >> 8
    return q


def _dequant64(fmt, q, O, I):
    """Closed form: the weights as float64, read from the block description."""
    if fmt == Z.FMT_TQ2:
        alpha = q[:O * 4].view(np.float32).astype(np.float64)
        c = q[O * 4:].reshape(O, I // 64, 16)
        w = np.concatenate([((c >> (2 * k)) & 3) for k in range(4)], axis=2).astype(np.float64) - 1
        return w.reshape(O, I) * alpha[:, None]
    if fmt == Z.FMT_Q4A:                            # tq2.h:269-282: w = d q + m
        grp = q.reshape(O * (I // 64), 36)
        d = grp[:, 0:2].copy().view(np.float16).astype(np.float64)
        m = grp[:, 2:4].copy().view(np.float16).astype(np.float64)
        h0, h1 = grp[:, 4:20], grp[:, 20:36]
        v = np.concatenate([h0 & 15, h0 >> 4, h1 & 15, h1 >> 4], axis=1).astype(np.float64)
        return (v * d + m).reshape(O, I)
    bb = 18 if fmt == Z.FMT_Q40 else 34
    blk = q.reshape(O * (I // 32), bb)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)
    if fmt == Z.FMT_Q40:
        v = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4], axis=1).astype(np.float64) - 8
    else:
        v = blk[:, 2:].view(np.int8).astype(np.float64)
    return (v * d).reshape(O, I)


def _matmul(fmt, W, x, O, I):
    L = Z.oracle()
    S = x.shape[0]
    y = np.zeros((S, O), np.float32)
    L.orc_matmul_f32(fmt, Z.ptr(y), Z.ptr(W), Z.ptr(np.ascontiguousarray(x, np.float32)), O, I, S)
    return y


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.array_equal(np.isnan(a), np.isnan(b)) and
                np.array_equal(a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32)))


def test_f32_dots_golden():
    """orc_q40/q80/tq2_dot_f32 and orc_matmul_f32 (tq2: alphas first, gpu.h:78-83)
    against the compiled reference's q40_dot_f32 / q80_dot_f32 / tq2_dot_f32
    (q40.h:290-305, 443-455, tq2.h:235-252) on the test_q40.c LCG stream."""
    g = np.load(os.path.join(GOLDEN, "kernels_lcg12345.npz"))
    L = Z.oracle()
    O, I, It = 16, 2816, 2048
    x = g["x"]
    for t in range(4):
        xt = np.ascontiguousarray(x[t])
        a = [L.orc_q40_dot_f32(Z.ptr(g["q40"][o * 88 * 18:]), Z.ptr(xt), I) for o in range(O)]
        b = [L.orc_q80_dot_f32(Z.ptr(g["q80"][o * 88 * 34:]), Z.ptr(xt), I) for o in range(O)]
        assert _bits_equal(a, g["d40f"][t]) and _bits_equal(b, g["d80f"][t])
    assert _bits_equal(_matmul(Z.FMT_Q40, g["q40"], x, O, I), g["d40f"])
    assert _bits_equal(_matmul(Z.FMT_Q80, g["q80"], x, O, I), g["d80f"])
    cb = g["tq"][O * 4:]
    c = [L.orc_tq2_dot_f32(Z.ptr(cb[o * (It // 4):]), C.c_float(g["alpha"][o]), Z.ptr(g["xt"]), It)
         for o in range(O)]
    assert _bits_equal(c, g["dtqf"])
    assert _bits_equal(_matmul(Z.FMT_TQ2, g["tq"], g["xt"].reshape(1, It), O, It)[0], g["dtqf"])
    qa = g["q4a"]                                   # q4a_dot_f32, tq2.h:405-427
    for t in range(4):
        xt = np.ascontiguousarray(x[t])
        a = [L.orc_q4a_dot_f32(Z.ptr(qa[o * 44 * 36:]), Z.ptr(xt), I) for o in range(O)]
        assert _bits_equal(a, g["dq4af"][t])
    assert _bits_equal(_matmul(Z.FMT_Q4A, qa, x, O, I), g["dq4af"])


@pytest.mark.parametrize("fmt", [Z.FMT_Q40, Z.FMT_Q80, Z.FMT_TQ2, Z.FMT_Q4A])
def test_f32_dots_closed_form(fmt):
    """The same dots against float64 dequant . x: every product is exact in
    double, so the two differ only by the summation order, far below one float
    ulp of the result plus the sum of magnitudes times 2^-50."""
    rng = np.random.default_rng(11 + fmt)
    O, S = 24, 3
    for I in (64, 704, 2048):
        if fmt == Z.FMT_TQ2:
            codes = rng.integers(0, 3, size=(O, I)).astype(np.int8)
            W = Z.tq2_tensor(codes, (rng.random(O) * 0.05 + 0.001).astype(np.float32))
        elif fmt == Z.FMT_Q4A:
            W = Z.q4a_rows(rng, O, I)
        else:
            W = _f32_rows(rng, fmt, O, I)
        x = rng.standard_normal((S, I)).astype(np.float32)
        x[1] *= np.float32(1e3)
        w64 = _dequant64(fmt, W, O, I)
        ref = x.astype(np.float64) @ w64.T
        mag = np.abs(x.astype(np.float64)) @ np.abs(w64).T
        got = _matmul(fmt, W, x, O, I).astype(np.float64)
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got - ref) <= ulp + mag * 2.0 ** -50), (fmt, I)


def test_f32_dots_vs_compiled_reference():
    """Live against the reference's own *_dot_f32 (oracle/_ref), on random rows whose
    fp16 scales include NaN, +-inf, -0 and subnormals, bit for bit."""
    R = Z.ref_lib("kernels")
    if R is None:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    for n in ("ref_q40_dot_f32", "ref_q80_dot_f32", "ref_tq2_dot_f32", "ref_q4a_dot_f32"):
        getattr(R, n).restype = C.c_float
    L = Z.oracle()
    rng = np.random.default_rng(29)
    for I in (32, 96, 2816):
        O = 16
        x = (rng.standard_normal((2, I)) * np.float32(3.0)).astype(np.float32)
        for fmt, bb, fo, fr in ((Z.FMT_Q40, 18, L.orc_q40_dot_f32, R.ref_q40_dot_f32),
                                (Z.FMT_Q80, 34, L.orc_q80_dot_f32, R.ref_q80_dot_f32)):
            W = _f32_rows(rng, fmt, O, I, specials=True)
            want = np.array([[fr(Z.ptr(W[o * (I // 32) * bb:]), Z.ptr(x[s]), I) for o in range(O)]
                             for s in range(2)], np.float32)
            got = np.array([[fo(Z.ptr(W[o * (I // 32) * bb:]), Z.ptr(x[s]), I) for o in range(O)]
                            for s in range(2)], np.float32)
            assert _bits_equal(got, want), (fmt, I)
            assert _bits_equal(_matmul(fmt, W, x, O, I), want), (fmt, I)
            assert np.isnan(want).any()
    for I in (64, 2048):
        O = 8
        codes = rng.integers(0, 3, size=(O, I)).astype(np.int8)
        alpha = (rng.standard_normal(O) * 0.05).astype(np.float32)
        alpha[0], alpha[1] = np.inf, 0.0
        W = Z.tq2_tensor(codes, alpha)
        x = rng.standard_normal((1, I)).astype(np.float32)
        cb = W[O * 4:]
        want = np.array([R.ref_tq2_dot_f32(Z.ptr(cb[o * (I // 4):]), C.c_float(alpha[o]), Z.ptr(x[0]), I)
                         for o in range(O)], np.float32)
        assert _bits_equal(_matmul(Z.FMT_TQ2, W, x, O, I)[0], want)
    for I in (64, 2048, 2816):
        O = 16
        W = Z.q4a_rows(rng, O, I, specials=True)
        x = (rng.standard_normal((2, I)) * np.float32(3.0)).astype(np.float32)
        want = np.array([[R.ref_q4a_dot_f32(Z.ptr(W[o * (I // 64) * 36:]), Z.ptr(x[s]), I)
                          for o in range(O)] for s in range(2)], np.float32)
        assert _bits_equal(_matmul(Z.FMT_Q4A, W, x, O, I), want), I
        assert np.isnan(want).any()


def test_tq2_layout_from_description():
    """tests/test_tq2.c:28-35: code j lives in byte j%16 of group j/64 at bit
    2*((j/16)%4); the oracle's packer and dequant must agree with that reading."""
    rng = np.random.default_rng(12345)
    for I in (64, 128, 512, 1792, 2048):
        c = rng.integers(0, 3, size=(1, I)).astype(np.int8)
        t = Z.tq2_tensor(c, np.array([0.25], np.float32))[4:]
        j = np.arange(I)
        read = (t[(j // 64) * 16 + j % 16] >> (2 * ((j // 16) % 4))) & 3
        assert np.array_equal(read, c[0])
        w = np.zeros(I, np.float32)
        L = Z.oracle()
        L.orc_tq2_dequant_row.argtypes = [Z.u8p, C.c_float, Z.f32p, C.c_int]
        L.orc_tq2_dequant_row(Z.ptr(t), 0.25, Z.ptr(w), I)
        assert np.array_equal(w, 0.25 * (c[0] - 1).astype(np.float32))


def test_tq2_sx_identity():
    """tq2.h:29-37: <c-1, x> = <c, x> - sum(x); Sx = sum_b sx_b * sum_j xq."""
    L = Z.oracle()
    rng = np.random.default_rng(5)
    I = 2048
    x = rng.standard_normal(I).astype(np.float32)
    q = np.zeros(I, np.int8)
    s = np.zeros(I // 32, np.float32)
    tot = L.orc_tq2_quant_act(Z.ptr(x), Z.ptr(q), Z.ptr(s), I)
    want = (s.astype(np.float64) * q.reshape(-1, 32).sum(1)).sum()
    assert abs(tot - want) <= 1e-6 * (abs(want) + 1)
    codes = np.ones((1, I), np.int8)                 # all-zero weights
    t = Z.tq2_tensor(codes, np.array([0.5], np.float32))
    v = L.orc_tq2_dot(Z.ptr(t[4:]), C.c_float(0.5), Z.ptr(q), Z.ptr(s), C.c_float(tot), I)
    assert abs(v) <= 1e-6 * abs(tot) + 1e-7


# ----------------------------------------------------------- routers (A10-A12)
@pytest.mark.parametrize("kind", ["gemma", "lfm", "maple"])
def test_router_matches_argsort_with_lower_index_ties(kind, layer_cache):
    L = layer_cache(kind, seed=11, E=32)
    x = Z.make_input(L, 16, 11)
    r = Z.oracle_moe(L, x, dump=True)
    K = L.K
    for s in range(16):
        lg = r.dump["logits"][s].astype(np.float64)
        if kind == "lfm":
            sg = 1.0 / (1.0 + np.exp(-lg.astype(np.float32)).astype(np.float32))
            lg = (sg.astype(np.float32) + L.bias).astype(np.float32).astype(np.float64)
        order = sorted(range(L.E), key=lambda e: (-lg[e], e))[:K]
        assert list(r.eidx[s * K:(s + 1) * K]) == order


def test_router_exact_ties_keep_lower_index(layer_cache):
    """Duplicate router rows give bit-identical logits; the insertion rule
    (gemma4.c:603-606, strict '>') keeps the lower expert index first."""
    L0 = layer_cache("maple", seed=12, E=16)
    L = Z.make_layer("maple", seed=12, E=16)
    L.router = L0.router.copy()
    L.router[9] = L.router[2]
    L.router[14] = L.router[2]
    x = Z.make_input(L, 32, 12)
    r = Z.oracle_moe(L, x, dump=True)
    for s in range(32):
        ids = list(r.eidx[s * L.K:(s + 1) * L.K])
        for a, b in ((2, 9), (2, 14), (9, 14)):
            if a in ids and b in ids:
                assert ids.index(a) < ids.index(b)


def test_dispatch_is_stable_counting_sort(layer_cache):
    L = layer_cache("gemma", seed=2, E=16)
    x = Z.make_input(L, 40, 13)
    r = Z.oracle_moe(L, x)
    S, K, nu = 40, L.K, len(r.uniq)
    offs = np.zeros(nu + 1, np.int32)
    rows = np.zeros(S * K, np.int32)
    wts = np.zeros(S * K, np.float32)
    slots = np.zeros(S * K, np.int32)
    Z.oracle().orc_dispatch(Z.ptr(r.eidx), Z.ptr(r.ewt), S, K, Z.ptr(r.uniq), nu, Z.ptr(offs),
                            Z.ptr(rows), Z.ptr(wts), Z.ptr(slots))
    flat = np.arange(S * K)
    for u, e in enumerate(r.uniq):
        sel = flat[r.eidx == e]                           # ascending flat index
        assert np.array_equal(rows[offs[u]:offs[u + 1]], sel // K)
        assert np.array_equal(slots[offs[u]:offs[u + 1]], sel % K)
    first = [int(np.argmax(r.eidx == e)) for e in r.uniq]
    assert first == sorted(first)                         # first-seen union order


# ------------------------------------------------------------- whole layers
# whole-MoE-layer fixtures (the kernel vectors and the gemma block/stack fixture have
# their own tests)
CASES = sorted(f[:-4] for f in os.listdir(GOLDEN)
               if f.endswith(".npz") and not f.startswith(("kernels", "gemma_block", "gemma_flash", "gemma_zipf")))


def load_case(name):
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    kw = {}
    if int(g["kw_E"]) > 0:
        kw["E"] = int(g["kw_E"])
    if int(g["kw_fmts"][0]) > 0:
        kw["fmts"] = tuple(int(v) for v in g["kw_fmts"])
    return g, str(g["kind"]), int(g["seed"]), kw, int(g["S"]), int(g["xseed"])


@pytest.mark.parametrize("name", CASES)
def test_layer_golden_bit_exact(name, layer_cache):
    """The oracle reproduces the compiled reference's layer bit for bit: ids, union
    order, weights and the f32 outputs."""
    from golden.make_golden import input_digest
    g, kind, seed, kw, S, xseed = load_case(name)
    L = layer_cache(kind, seed=seed, **kw)
    x = Z.make_input(L, S, xseed)
    assert input_digest(L, x) == str(g["digest"]), "input generator drifted from the fixture"
    r = Z.oracle_moe(L, x)
    assert np.array_equal(r.eidx, g["eidx"])
    assert np.array_equal(r.uniq, g["uniq"])
    assert np.array_equal(r.ewt.view(np.uint32), g["ewt"].view(np.uint32))
    assert np.array_equal(r.out.view(np.uint32), g["out"].view(np.uint32))


@pytest.mark.parametrize("kind,kw,S", [("gemma", dict(E=24, D=1024, MI=512), 33),
                                       ("lfm", dict(E=12, fmts=(2, 2, 2), D=1024, MI=768), 17),
                                       ("maple", dict(E=40, D=1024, MI=512), 29),
                                       ("ling", dict(E=64, D=1024, MI=256), 40),
                                       ("ling", dict(E=128, D=512, MI=128, fmts=(2, 2, 2)), 9)])
def test_layer_vs_compiled_reference(kind, kw, S):
    """Live diff against oracle/_ref at shapes the fixtures do not cover."""
    if Z.ref_lib("gemma4") is None:
        pytest.skip("oracle/_ref not built here")
    L = Z.make_layer(kind, seed=21, **kw)
    x = Z.make_input(L, S, 21)
    a, b = Z.oracle_moe(L, x), Z.ref_moe(L, x)
    assert np.array_equal(a.eidx, b.eidx) and np.array_equal(a.uniq, b.uniq)
    assert np.array_equal(a.out.view(np.uint32), b.out.view(np.uint32))


def test_fp32_tier_tolerance_is_discriminating(layer_cache):
    """The GPU tier's 1e-3 relative-L2 bound must reject a plausible slip: dropping
    one expert's contribution, or using silu for gemma's GeGLU."""
    L = layer_cache("gemma", seed=2, E=16)
    x = Z.make_input(L, 8, 14)
    good = Z.oracle_moe(L, x).out
    L2 = Z.make_layer("gemma", seed=2, E=16)
    L2.act = Z.ACT_SWIGLU
    bad = Z.oracle_moe(L2, x).out
    assert Z.rel_l2(bad, good) > 1e-2
    L3 = Z.make_layer("gemma", seed=2, E=16, K=7)
    assert Z.rel_l2(Z.oracle_moe(L3, x).out, good) > 1e-2


def test_ling_grouped_router_keeps_only_live_groups():
    """A13 (ling.c:705-789): every selected expert lies in one of topk_group groups,
    and those groups are the ones with the largest top-2 biased scores (recomputed
    here in numpy from the oracle's own logits, lower group on ties)."""
    L = Z.make_layer("ling", seed=31, E=128, D=512, MI=128)
    x = Z.make_input(L, 24, 31)
    r = Z.oracle_moe(L, x, dump=True)
    EG = L.E // L.n_group
    for s_ in range(24):
        v = r.dump["logits"][s_].astype(np.float32)
        sg = (np.float32(1) / (np.float32(1) + np.exp(-v).astype(np.float32))).astype(np.float32)
        sel = (sg + L.bias).astype(np.float32)
        top2 = np.sort(sel.reshape(L.n_group, EG), axis=1)[:, -2:]
        gs = (top2[:, 1] + top2[:, 0]).astype(np.float32)
        keep = sorted(range(L.n_group), key=lambda g: (-gs[g], g))[:L.topk_group]
        ids = r.eidx[s_ * L.K:(s_ + 1) * L.K]
        assert set(int(e) // EG for e in ids) <= set(keep)
        live = np.concatenate([np.arange(g * EG, (g + 1) * EG) for g in keep])
        want = sorted(live, key=lambda e: (-sel[e], e))[:L.K]
        assert list(ids) == want


def test_tensor_sizes():
    """tests/test_tq2.c size arithmetic, with q40.h:313-314 / 461-462 for the block
    formats: the byte counts gpu_matmul checks a tensor's mapping against."""
    L = Z.oracle()
    for I in (64, 128, 512, 1792, 2048, 2816):
        assert L.orc_tensor_bytes(Z.FMT_TQ2, 7, I) == 7 * 4 + 7 * (I // 4)
        assert L.orc_tensor_bytes(Z.FMT_Q4A, 7, I) == 7 * (I // 64) * 36
        assert L.orc_tensor_bytes(Z.FMT_Q40, 7, I) == 7 * (I // 32) * 18
        assert L.orc_tensor_bytes(Z.FMT_Q80, 7, I) == 7 * (I // 32) * 34
        for f in (Z.FMT_Q40, Z.FMT_Q80, Z.FMT_TQ2, Z.FMT_Q4A):
            assert L.orc_tensor_bytes(f, 7, I) == Z.tensor_bytes(f, 7, I)


# ------------------------------------------- the gemma Zipf offset
def _route_oracle(D, E, K, router, rscale, pes, bias, x):
    cfg = Z.OrcCfg(D, 64, E, K, Z.GATE_GEMMA, Z.ACT_GEGLU_TANH, 1, 1, 1, 1,
                   0 if bias is None else 1, 0.0, 1.0, 7.0, 1, 1)
    w = Z.OrcWeights(Z.ptr(router), Z.ptr(rscale), Z.ptr(pes), Z.ptr(bias), None, None, None, 0)
    S = x.shape[0]
    ids = np.zeros((S, K), np.int32)
    wts = np.zeros((S, K), np.float32)
    lg = np.zeros((S, E), np.float32)
    for s in range(S):
        Z.oracle().orc_route(C.byref(cfg), C.byref(w), Z.ptr(np.ascontiguousarray(x[s])), Z.ptr(ids[s]),
                             Z.ptr(wts[s]), Z.ptr(lg[s]))
    return ids, wts, lg


def _route_ref(D, E, K, router, rscale, pes, x):
    R = Z.ref_lib("gemma4")
    R.ref_g4_route.argtypes = [C.c_int, C.c_int, C.c_int, C.c_float, Z.f32p, Z.f32p, Z.f32p, Z.f32p,
                               Z.i32p, Z.f32p]
    S = x.shape[0]
    ids = np.zeros((S, K), np.int32)
    wts = np.zeros((S, K), np.float32)
    for s in range(S):
        assert R.ref_g4_route(D, E, K, 0.0, Z.ptr(router), Z.ptr(rscale), Z.ptr(pes),
                              Z.ptr(np.ascontiguousarray(x[s])), Z.ptr(ids[s]), Z.ptr(wts[s])) == 0
    return ids, wts


ZIPF_PAD = 32


def _zipf_route_case(D=1024, E=32, K=8, S=24, seed=51):
    """The oracle's biased router at D against the reference's unbiased route_row at
    D' = D + 32 (gemma4.c:581-613), the offset carried by the last extra element.

    With every input element +-1 and eps = 0 both rmsnorm factors are exactly 1
    (gemma4.c:428). The reference's router inputs are c_i = fl(rscale'_i * rs') with
    rs' = 1/sqrtf(D'); the oracle gets rscale_i = 32 c_i, so at rs = 1/sqrtf(1024)
    = 1/32 its inputs are the same c_i. Extra elements D .. D'-2 have router weight 0
    (each adds an exact +0). The last (x = 1, rscale' = 1) is rs' exactly, and its
    router weight q_e = fl(zipf_e / rs') makes the reference's last product
    bias_e = fl(q_e * rs'). The reference's logit is then fl(chain_D + bias_e): the
    offset added once, after the chain. D' stays a multiple of 32: the compiled
    reference adds its vectorised products unfused, but fuses the scalar remainder
    of the loop (the last D' mod 4 products), which a D + 1 layout would hit."""
    assert D == 1024
    P = ZIPF_PAD
    rng = np.random.default_rng(seed)
    rsr = np.float32(1.0) / np.sqrt(np.float32(D + P))
    rsc_ref = np.ones(D + P, np.float32)
    rsc_ref[:D] = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    c = (rsc_ref[:D] * rsr).astype(np.float32)
    rsc = (c * np.float32(32)).astype(np.float32)
    router = rng.standard_normal((E, D), dtype=np.float32)
    zipf = (-1.1 * np.log(rng.permutation(E) + 1)).astype(np.float32)
    q = (zipf / rsr).astype(np.float32)
    bias = (q * rsr).astype(np.float32)
    router_ref = np.zeros((E, D + P), np.float32)
    router_ref[:, :D] = router
    router_ref[:, D + P - 1] = q
    pes = (1 + 0.1 * rng.random(E)).astype(np.float32)
    x = Z.pm1_input(S, D, seed, last_one=False)
    x_ref = np.ascontiguousarray(np.concatenate([x, np.ones((S, P), np.float32)], axis=1))
    return D, E, K, router, rsc, pes, bias, x, router_ref, rsc_ref, x_ref


def test_gemma_zipf_offset_equals_reference_last_product():
    """The Zipf-offset branch (zz_oracle.c, gemma) equals the compiled reference bit for
    bit: ids and softmax weights, which both see the offset logits. Its logits are
    fl(unbiased chain + offset), and its ids a lower-index-tie argsort of them."""
    if Z.ref_lib("gemma4") is None:
        pytest.skip("oracle/_ref not built here")
    D, E, K, router, rsc, pes, bias, x, router_ref, rsc_ref, x_ref = _zipf_route_case()
    ids, wts, lg = _route_oracle(D, E, K, router, rsc, pes, bias, x)
    rid, rwt = _route_ref(D + ZIPF_PAD, E, K, router_ref, rsc_ref, pes, x_ref)
    assert np.array_equal(ids, rid)
    assert np.array_equal(wts.view(np.uint32), rwt.view(np.uint32))
    _, _, lg0 = _route_oracle(D, E, K, router, rsc, pes, None, x)
    assert np.array_equal(lg.view(np.uint32), (lg0 + bias).astype(np.float32).view(np.uint32))
    for s in range(x.shape[0]):
        assert list(ids[s]) == sorted(range(E), key=lambda e: (-float(lg[s, e]), e))[:K]
    # the offset moves the choice: the pin is not vacuous
    ids0, _, _ = _route_oracle(D, E, K, router, rsc, pes, None, x)
    assert not np.array_equal(ids0, ids)


@pytest.mark.parametrize("plant", [1, 2, 3, 4])
def test_gemma_zipf_offset_pin_rejects_planted_slips(plant):
    """Each plausible slip in the offset branch fails the reference pin: the offset as
    the chain's first term (1), before the chain's last product (2), in the softmax
    only (3), in the selection only (4)."""
    if Z.ref_lib("gemma4") is None:
        pytest.skip("oracle/_ref not built here")
    D, E, K, router, rsc, pes, bias, x, router_ref, rsc_ref, x_ref = _zipf_route_case()
    rid, rwt = _route_ref(D + ZIPF_PAD, E, K, router_ref, rsc_ref, pes, x_ref)
    Z.oracle().orc_set_plant(plant)
    try:
        ids, wts, _ = _route_oracle(D, E, K, router, rsc, pes, bias, x)
    finally:
        Z.oracle().orc_set_plant(0)
    assert not (np.array_equal(ids, rid) and np.array_equal(wts.view(np.uint32), rwt.view(np.uint32)))


def test_gemma_zipf_layer_golden():
    """A whole Zipf-offset layer at the Gemma-4 shape (configs[1]: D=2816, 128 experts,
    top-8) bit for bit against the fixture the compiled reference wrote, with the
    offset in the reference's last router column (zzref.zipf_pin_case)."""
    from golden.make_golden import input_digest
    g = np.load(os.path.join(GOLDEN, "gemma_zipf_e128_s8.npz"))
    Lo, Lr, x = Z.zipf_pin_case(**Z.ZIPF_PIN)
    assert input_digest(Lr, x) == str(g["digest"]), "input generator drifted from the fixture"
    r = Z.oracle_moe(Lo, x)
    assert np.array_equal(r.eidx, g["eidx"])
    assert np.array_equal(r.uniq, g["uniq"])
    assert np.array_equal(r.ewt.view(np.uint32), g["ewt"].view(np.uint32))
    assert np.array_equal(r.out.view(np.uint32), g["out"].view(np.uint32))
    if Z.ref_lib("gemma4") is not None:        # and live
        b = Z.ref_moe(Lr, x)
        assert np.array_equal(b.eidx, g["eidx"]) and np.array_equal(b.out.view(np.uint32), g["out"].view(np.uint32))


# ------------------------------------------------------------ q8_0 dequant (A7)
def _q80_rows(rng, O, I):
    q = Z.quant_rows(Z.FMT_Q80, (rng.standard_normal((O, I)) * 0.05).astype(np.float32)).reshape(-1, 34)
    # special scales: NaN, +-inf, -0, subnormal halves
    for k, h in enumerate([0x7e00, 0x7c00, 0xfc00, 0x8000, 0x0001, 0x03ff]):
        q[3 * k + 1, 0], q[3 * k + 1, 1] = h & 255, h >> 8
    return q.reshape(-1)


def test_q80_dequant_matches_reference_and_closed_form():
    """orc_q80_dequant_row (q40.h:349-356) against numpy (fp16 scale times the int8
    code, one float rounding) and the compiled reference's q80_dequant_row."""
    L = Z.oracle()
    L.orc_q80_dequant_row.argtypes = [Z.u8p, Z.f32p, C.c_int]
    rng = np.random.default_rng(61)
    O, I = 8, 2816
    q = _q80_rows(rng, O, I)
    got = np.zeros(O * I, np.float32)
    L.orc_q80_dequant_row(Z.ptr(q), Z.ptr(got), O * I)
    blk = q.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    with np.errstate(invalid="ignore"):              # inf * 0
        want = (d * blk[:, 2:].view(np.int8).astype(np.float32)).astype(np.float32).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    R = Z.ref_lib("kernels")
    if R is not None:
        ref = np.zeros(O * I, np.float32)
        R.ref_q80_dequant_row.argtypes = [Z.u8p, Z.f32p, C.c_int]
        R.ref_q80_dequant_row(Z.ptr(q), Z.ptr(ref), O * I)
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    L.orc_set_plant(5)
    try:
        bad = np.zeros(O * I, np.float32)
        L.orc_q80_dequant_row(Z.ptr(q), Z.ptr(bad), O * I)
    finally:
        L.orc_set_plant(0)
    assert not np.array_equal(bad[fin].view(np.uint32), want[fin].view(np.uint32))
