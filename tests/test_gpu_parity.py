"""GPU parity: libzzmoe.so on an MI355X against the oracle and the golden vectors
the compiled reference wrote. Calls go through the C ABI (zunzuncito_amd is a
ctypes binding of include/zz_moe.h and include/zz_gpu.h).

Tiers:
  bit-exact  routing ids and order, union order, dispatch lists, the int8
             activations and scales, the per-block int32 dots;
  fp32       layer outputs within 1e-3 relative L2, gate weights within 1e-4.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import zzref as Z
import zunzuncito_amd as zz
from test_oracle import CASES, load_case

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-3          # fp32 tier: relative L2 of the layer output
WT_RTOL = 1e-4          # gate weights (softmax/sigmoid of certified logits)


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def dev():
    name = zz.init()            # raises: no silent CPU path
    return name


def gpu_layer(L):
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, L.bias, L.pre_ln, L.post_ln, norm_topk=L.norm_topk,
                    use_bias=L.use_bias, eps=L.eps, routed_scaling=L.routed_scaling,
                    clamp=L.clamp, n_group=L.n_group, topk_group=L.topk_group)
    m.upload_all(L.experts)
    return m


def check_layer(m, L, x, want, dump=False):
    out, eidx, ewt = m.forward(x)
    assert np.array_equal(eidx, want.eidx), "routing ids differ"
    np.testing.assert_allclose(ewt, want.ewt, rtol=WT_RTOL, atol=1e-6)
    err = Z.rel_l2(out, want.out)
    assert err < OUT_TOL, err
    return out, eidx, ewt, err


def test_device(dev):
    say("device:", dev)
    assert "gfx950" in dev


@pytest.mark.parametrize("name", CASES)
def test_golden_layer(dev, name, layer_cache):
    g, kind, seed, kw, S, xseed = load_case(name)
    say("case", name)
    L = layer_cache(kind, seed=seed, **kw)
    x = Z.make_input(L, S, xseed)
    m = gpu_layer(L)
    try:
        want = Z.MoeResult(g["out"], g["eidx"], g["ewt"], g["uniq"])
        out, eidx, ewt, err = check_layer(m, L, x, want)
        say(f"  out rel L2 {err:.2e}")
        # integer tier on the dump of that forward
        orc = Z.oracle_moe(L, x, dump=True)
        d = m.debug(S)
        assert np.array_equal(d["xq"], orc.dump["xq"])
        assert np.array_equal(d["xs"].view(np.uint32), orc.dump["xs"].view(np.uint32))
        assert np.array_equal(d["uniq"], g["uniq"])
        offs = np.zeros(len(g["uniq"]) + 1, np.int32)
        rows = np.zeros(S * L.K, np.int32)
        slots = np.zeros(S * L.K, np.int32)
        Z.oracle().orc_dispatch(Z.ptr(orc.eidx), Z.ptr(orc.ewt), S, L.K, Z.ptr(orc.uniq),
                                len(orc.uniq), Z.ptr(offs), Z.ptr(rows), None, Z.ptr(slots))
        assert np.array_equal(d["offs"], offs)
        assert np.array_equal(d["rows"], rows) and np.array_equal(d["slots"], slots)
        # the hidden goes through tanhf/expf, whose device and glibc results may
        # differ by an ulp: its int8 codes agree except for rare +-1 flips
        diff = np.abs(d["hq"].astype(np.int32) - orc.dump["hq"].astype(np.int32))
        assert diff.max() <= 1 and (diff > 0).mean() < 2e-3, (diff.max(), (diff > 0).mean())
    finally:
        m.close()


def test_golden_zipf_layer(dev):
    """configs[1]'s Zipf-offset routing at the Gemma-4 shape against the fixture the
    compiled reference wrote (its last router column carries the offset exactly,
    zzref.zipf_pin_case): the batch on the matrix-core path and each token alone on
    the decode path. Ids exact, outputs within the fp32 tier."""
    g = np.load(os.path.join(Z.ROOT, "tests", "golden", "gemma_zipf_e128_s8.npz"))
    Lo, _, x = Z.zipf_pin_case(**Z.ZIPF_PIN)
    m = gpu_layer(Lo)
    try:
        K = Lo.K
        want = Z.MoeResult(g["out"], g["eidx"], g["ewt"], g["uniq"])
        say("case zipf S=8")
        _, _, _, err = check_layer(m, Lo, x, want)
        assert np.array_equal(m.debug(x.shape[0])["uniq"], g["uniq"])
        say(f"  out rel L2 {err:.2e}")
        for s in range(x.shape[0]):
            say(f"case zipf token {s} (S=1)")
            w1 = Z.MoeResult(g["out"][s:s + 1], g["eidx"][s * K:(s + 1) * K], g["ewt"][s * K:(s + 1) * K], None)
            check_layer(m, Lo, x[s:s + 1], w1)
    finally:
        m.close()


# D % 256 == 0 takes 256-wide K chunks, other D % 64 == 0 the 64-wide ones
@pytest.mark.parametrize("kind,kw,S", [
    ("gemma", dict(), 64), ("gemma", dict(zipf=True, E=64), 37), ("gemma", dict(D=1088, E=64), 16),
    ("lfm", dict(), 48), ("lfm", dict(D=1088), 20), ("maple", dict(E=16), 32),
    ("ling", dict(), 64), ("ling", dict(D=1088, MI=256), 17)])
def test_exact_router_logits(dev, kind, kw, S, layer_cache):
    """At S >= 16 the batched router logits are the reference's own serial chains, bit
    for bit: gemma's unfused fp32 chain (+ the bias), lfm/maple's double chain and
    ling's eight double accumulators, each rounded to float as the reference does."""
    L = layer_cache(kind, seed=3, **kw)
    say("case", kind, kw, "S", S)
    x = Z.make_input(L, S, 5)
    m = gpu_layer(L)
    try:
        m.forward(x)
        got = m.debug(S, logits=True)["logits"]
        want = Z.oracle_moe(L, x, dump=True).dump["logits"]
        assert np.array_equal(got.astype(np.float32).astype(np.float64), got), "not float-valued"
        bad = got.astype(np.float32).view(np.uint32) != want.view(np.uint32)
        assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:4])
    finally:
        m.close()


@pytest.mark.parametrize("kind,kw", [("gemma", dict(E=8)), ("lfm", dict(E=8)),
                                     ("maple", dict(E=8, D=1024, MI=512))])
def test_blockdots_bit_exact(dev, kind, kw, layer_cache):
    """Per-block int32 dots of every tensor of an expert (q4_0, q8_0, tq2) against the
    oracle's brute-force dots, on quantised activations of both signs and saturating
    extremes."""
    say("blockdots", kind)
    L = layer_cache(kind, seed=31, **kw)
    m = gpu_layer(L)
    try:
        rng = np.random.default_rng(31)
        g, u, d = L.tensor_sizes()
        for eid in (0, L.E - 1):
            rec = L.experts[eid * L.esz:(eid + 1) * L.esz]
            for t, (off, (O, I)) in enumerate(zip((0, g, g + u), ((L.MI, L.D), (L.MI, L.D), (L.D, L.MI)))):
                fmt = L.fmts[t]
                xq = rng.integers(-127, 128, I, dtype=np.int8)
                xq[:32] = 127
                xq[32:64] = -127
                rows = np.arange(O)[:: max(1, O // 96)][:96]
                got = m.blockdots(eid, t, 0, O, xq)
                T = rec[off:off + Z.tensor_bytes(fmt, O, I)]
                for r in rows:
                    if fmt == Z.FMT_TQ2:
                        row = T[O * 4 + r * (I // 4):]
                    else:
                        row = T[r * (I // 32) * (18 if fmt == Z.FMT_Q40 else 34):]
                    want = np.zeros(I // 32, np.int32)
                    Z.oracle().orc_blockdots(fmt, Z.ptr(np.ascontiguousarray(row)), Z.ptr(xq), I,
                                             Z.ptr(want))
                    assert np.array_equal(got[r], want), (eid, t, r)
    finally:
        m.close()


_A, _C = 6364136223846793005, 1442695040888963407


def lcg64_stream(r0, n, lanes=1 << 16):
    """States r_1..r_n of r <- r*A + C (mod 2^64) from r_0, vectorised by jumping
    `lanes` steps at a time: r_{i+L} = A^L r_i + C (A^L - 1)/(A - 1)."""
    M = 2 ** 64
    first = np.empty(min(lanes, n), np.uint64)
    r = r0
    for i in range(first.size):
        r = (r * _A + _C) % M
        first[i] = r
    if n <= lanes:
        return first[:n]
    aL, cL = 1, 0
    for _ in range(lanes):                       # compose the affine map L times
        aL, cL = (aL * _A) % M, (cL * _A + _C) % M
    out = np.empty(((n + lanes - 1) // lanes) * lanes, np.uint64)
    cur = first.copy()
    with np.errstate(over="ignore"):
        for k in range(out.size // lanes):
            out[k * lanes:(k + 1) * lanes] = cur
            cur = cur * np.uint64(aL) + np.uint64(cL)
    return out[:n]


def _lcg_check_gpu(O, I, t):
    """gemma4.c:2335-2343: W bytes then x from the reference's 64-bit LCG."""
    wb = O * (I // 32) * 18
    st = lcg64_stream((0x243f6a8885a308d3 ^ t) % 2 ** 64, wb + I)
    W = ((st[:wb] >> np.uint64(40)) & np.uint64(0xff)).astype(np.uint8)
    xi = (st[wb:] >> np.uint64(40)).astype(np.int64) - 8388608
    x = (xi.astype(np.float32) / np.float32(8388608.0)).astype(np.float32)
    return W, x


@pytest.mark.parametrize("t,O,I", [(0, 4096, 2816), (1, 8192, 2816), (2, 2112, 2816),
                                   (3, 2816, 2112), (4, 704, 2816), (5, 2816, 704)])
def test_check_gpu_shapes(dev, t, O, I):
    """gemma4.c:2315-2368 --check-gpu: gpu_q40_matmul vs q40_dot_f32 at the engine's
    shapes, max|d| / max|ref| < 1e-4 over the finite rows. Rows whose random fp16
    scale is NaN or inf must be non-finite in the same way (NaN where the reference
    has NaN, the same infinity otherwise): both scale each block's sum by d once."""
    say("check_gpu", O, I)
    W, x = _lcg_check_gpu(O, I, t)
    Wm = zz.gpu_map(W)
    y = np.zeros((1, O), np.float32)
    assert zz.lib().gpu_q40_matmul(y.ctypes.data_as(zz._f32p), Wm.ctypes.data_as(zz._u8p),
                                   x.ctypes.data_as(zz._f32p), O, I, 1) == 1
    ref = np.zeros((1, O), np.float32)
    Z.oracle().orc_matmul_f32(Z.FMT_Q40, Z.ptr(ref), Z.ptr(Wm), Z.ptr(x), O, I, 1)
    fin = np.isfinite(ref[0])
    assert np.array_equal(np.isfinite(y[0]), fin), "finite rows differ"
    nan = np.isnan(ref[0])
    assert np.array_equal(np.isnan(y[0]), nan), "NaN rows differ"
    assert np.array_equal(y[0][~fin & ~nan], ref[0][~fin & ~nan]), "infinite rows differ"
    rel = np.abs(y[0][fin] - ref[0][fin]).max() / (np.abs(ref[0][fin]).max() + 1e-9)
    say(f"  max rel err {rel:.3e}, {int((~fin).sum())} non-finite rows")
    assert rel < 1e-4


@pytest.mark.parametrize("fmt", [Z.FMT_Q80, Z.FMT_TQ2, Z.FMT_Q4A])
def test_gpu_matmul_other_formats(dev, fmt):
    rng = np.random.default_rng(41)
    O, I, S = 1792, 2048, 3
    if fmt == Z.FMT_TQ2:
        W = Z.make_expert_tq2(rng, O, I)
    elif fmt == Z.FMT_Q4A:
        W = Z.q4a_rows(rng, O, I)
    else:
        W = Z.quant_rows(fmt, (rng.standard_normal((O, I)) * 0.02).astype(np.float32))
    Wm = zz.gpu_map(W)
    x = rng.standard_normal((S, I)).astype(np.float32)
    y = zz.gpu_matmul(fmt, Wm, x, O, I)
    ref = np.zeros((S, O), np.float32)
    Z.oracle().orc_matmul_f32(fmt, Z.ptr(ref), Z.ptr(Wm), Z.ptr(x), O, I, S)
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-4


def test_gpu_map_slot_refill_is_seen(dev):
    """The engines map an expert slot once, while empty (gemma4.c:2051-2058), then
    pread other experts into the same bytes (gemma4.c:484-491). A discrete GPU copies
    at map time; gpu_matmul compares the tensor's sampled fingerprint with the one
    of its last upload and uploads it again when the host bytes changed, so an
    unchanged engine computes on the expert it just read. Unchanged bytes are not
    uploaded again, and an explicit re-map still refreshes a sub-range."""
    rng = np.random.default_rng(43)
    O, I = 256, 512
    rb = O * (I // 32) * 18
    slot = np.zeros(2 * rb, np.uint8)               # two tensors in one mapped slot
    A = Z.quant_rows(Z.FMT_Q40, (rng.standard_normal((O, I)) * 0.02).astype(np.float32))
    Bw = Z.quant_rows(Z.FMT_Q40, (rng.standard_normal((O, I)) * 0.02).astype(np.float32))
    Cw = Z.quant_rows(Z.FMT_Q40, (rng.standard_normal((O, I)) * 0.02).astype(np.float32))
    slot[:rb] = A
    slot[rb:] = Cw
    Wm = zz.gpu_map(slot)
    x = rng.standard_normal((1, I)).astype(np.float32)
    L = zz.lib()

    def ref(W):
        y = np.zeros((1, O), np.float32)
        Z.oracle().orc_matmul_f32(Z.FMT_Q40, Z.ptr(y), Z.ptr(np.ascontiguousarray(W)), Z.ptr(x), O, I, 1)
        return y

    def rel(y, W):
        return np.abs(y - ref(W)).max() / np.abs(ref(W)).max()

    n0 = L.zz_gpu_map_refreshes()
    assert rel(zz.gpu_matmul(Z.FMT_Q40, Wm[:rb], x, O, I), A) < 1e-4
    assert rel(zz.gpu_matmul(Z.FMT_Q40, Wm[rb:], x, O, I), Cw) < 1e-4
    assert L.zz_gpu_map_refreshes() == n0            # unchanged: nothing uploaded again
    Wm[:rb] = Bw                                    # the "pread" of another expert
    assert rel(zz.gpu_matmul(Z.FMT_Q40, Wm[:rb], x, O, I), Bw) < 1e-4
    assert L.zz_gpu_map_refreshes() == n0 + 1
    assert rel(zz.gpu_matmul(Z.FMT_Q40, Wm[rb:], x, O, I), Cw) < 1e-4
    assert L.zz_gpu_map_refreshes() == n0 + 1        # the other tensor was untouched
    Wm[:rb] = A
    assert L.gpu_map(C.c_void_p(Wm.ctypes.data), rb) == 1   # an explicit refresh
    assert rel(zz.gpu_matmul(Z.FMT_Q40, Wm[:rb], x, O, I), A) < 1e-4
    assert L.zz_gpu_map_refreshes() == n0 + 1


def test_gpu_matmul_declines_unmapped_and_bad_shapes(dev):
    """A refused call leaves y untouched: W outside every mapping, an unknown format,
    and a Q4A / TQ2 row length that is not a whole number of 64-groups."""
    x = np.ones((1, 64), np.float32)
    y = np.full((1, 8), 5.0, np.float32)
    W = np.zeros(8 * 2 * 18, np.uint8)               # never gpu_map'd
    L = zz.lib()
    assert L.gpu_matmul(1, y.ctypes.data_as(zz._f32p), W.ctypes.data_as(zz._u8p),
                        x.ctypes.data_as(zz._f32p), 8, 64, 1) == 0
    Wm = zz.gpu_map(np.zeros(8 * 64, np.uint8))
    for fmt, I in ((5, 64), (Z.FMT_Q4A, 32), (Z.FMT_TQ2, 32)):
        assert L.gpu_matmul(fmt, y.ctypes.data_as(zz._f32p), Wm.ctypes.data_as(zz._u8p),
                            x.ctypes.data_as(zz._f32p), 8, I, 1) == 0
    assert np.all(y == 5.0)


def _unit(v):
    """maple.c:1781 UNIT(): (float)((int64)(r >> 40) - 2^23) / 2^23."""
    return ((v >> np.uint64(40)).astype(np.int64) - 8388608).astype(np.float32) / np.float32(8388608.0)


@pytest.mark.parametrize("t,fmt,O,I", [(0, Z.FMT_TQ2, 2048, 2048), (1, Z.FMT_TQ2, 512, 2048),
                                       (3, Z.FMT_TQ2, 2048, 512), (4, Z.FMT_Q4A, 4096, 2048),
                                       (5, Z.FMT_Q4A, 4736, 2048)])
def test_maple_check_gpu_shapes(dev, t, fmt, O, I):
    """maple.c:1756-1826 --check-gpu: gpu_matmul vs the reference's w_dot_f32
    (tq2_dot_f32, q4a_dot_f32) at the engine's shapes, max|d| / max|ref| < 1e-4.
    Weights from the same 64-bit LCG: random bytes, then tq2 row scales or q4a
    group scales and biases overwritten, then x."""
    say("maple check_gpu", fmt, O, I)
    wb = Z.tensor_bytes(fmt, O, I)
    nsc = O if fmt == Z.FMT_TQ2 else 2 * O * (I // 64)
    st = lcg64_stream((0x243f6a8885a308d3 ^ t) % 2 ** 64, wb + nsc + I)
    W = ((st[:wb] >> np.uint64(40)) & np.uint64(0xff)).astype(np.uint8)
    u = _unit(st[wb:wb + nsc])
    if fmt == Z.FMT_TQ2:
        W[:4 * O] = (np.float32(0.01) + np.float32(0.04) * np.abs(u)).astype(np.float32).view(np.uint8)
    else:
        g = W.reshape(-1, 36)
        g[:, 0:2] = (np.float32(0.002) + np.float32(0.01) * np.abs(u[0::2])).astype(np.float16).view(np.uint8).reshape(-1, 2)
        g[:, 2:4] = (np.float32(0.05) * u[1::2]).astype(np.float16).view(np.uint8).reshape(-1, 2)
    x = _unit(st[wb + nsc:]).reshape(1, I)
    Wm = zz.gpu_map(W)
    y = zz.gpu_matmul(fmt, Wm, x, O, I)
    ref = np.zeros((1, O), np.float32)
    Z.oracle().orc_matmul_f32(fmt, Z.ptr(ref), Z.ptr(Wm), Z.ptr(x), O, I, 1)
    rel = np.abs(y - ref).max() / (np.abs(ref).max() + 1e-9)
    say(f"  max rel err {rel:.3e}")
    assert rel < 1e-4


def _item_buckets(eidx, E):
    """The FFN body each work item takes: <= 4 tokens "tiny" (4x4x4, one token set),
    5-8 "two-set" (4x4x4 with two sets, q4_0; other formats the 16-token body), else
    the number of 16-token tiles; experts of more than 64 tokens split into items."""
    seen = set()
    for c in np.bincount(eidx, minlength=E):
        for n in [64] * (c // 64) + [c % 64]:
            if n:
                seen.add("tiny" if n <= 4 else "two-set" if n <= 8 else (n + 15) // 16)
    return seen


@pytest.mark.parametrize("kind,kw,sizes", [
    ("gemma", dict(E=8, K=2), (12, 24, 100, 160, 200, 300)),
    # q4_0 gate/up and q8_0 down: items of 5-8 tokens take the two-set body for
    # gate/up and the 16-token body for down
    ("lfm", dict(E=8, K=2, D=1024, MI=512), (12, 24, 100, 200))])
def test_every_token_tile_count(dev, kind, kw, sizes, layer_cache):
    """Work items of every shape against the oracle: 8 experts and top-2 at S = 12 ..
    300 put 3 .. 80 tokens on an expert, so items of <= 4 tokens, of 5-8, of 1, 2, 3
    and 4 token tiles of 16, and experts split over two items all run."""
    L = layer_cache(kind, seed=11, **kw)
    m = gpu_layer(L)
    seen = set()
    try:
        for S in sizes:
            x = Z.make_input(L, S, 7)
            want = Z.oracle_moe(L, x)
            seen |= _item_buckets(want.eidx, L.E)
            say(f"case {kind} S={S}")
            out, eidx, ewt, err = check_layer(m, L, x, want)
            say(f"  S={S} out rel L2 {err:.2e}")
        need = {"tiny", "two-set", 1, 2, 3, 4} if kind == "gemma" else {"tiny", "two-set", 1}
        assert seen >= need, seen
    finally:
        m.close()


# --------------------------------------------------------------- BASELINE configs
def test_config2_gemma_zipf_s512(dev, layer_cache):
    """Config 2: S=512 prefill, Zipf(1.1) logit offsets (a harness extension that
    reduces to the reference at bias 0), skewed batch union."""
    say("config2 gemma zipf S=512")
    L = layer_cache("gemma", seed=2, zipf=True)
    x = Z.make_input(L, 512, 2)
    want = Z.oracle_moe(L, x)
    m = gpu_layer(L)
    try:
        out, eidx, ewt, err = check_layer(m, L, x, want)
        cnt = np.bincount(eidx, minlength=L.E)
        say(f"  nu {len(want.uniq)} max/min per-expert {cnt.max()}/{cnt.min()} rel L2 {err:.2e}")
        assert len(want.uniq) > 64 and cnt.max() > 4 * max(1, np.median(cnt))
        # a skewed union of many experts is placed whole: each expert's items on one XCD
        xcds = Z.check_items(m.debug(512))
        assert all(len(x) == 1 for x in xcds.values()), xcds
    finally:
        m.close()


@pytest.mark.parametrize("S", [1, 8, 256])
def test_config3_lfm_mixed(dev, S, layer_cache):
    """Config 3: LFM shape, gate/up q4_0 with down q8_0 (per-tensor formats)."""
    say("config3 lfm S", S)
    L = layer_cache("lfm", seed=3)
    x = Z.make_input(L, S, 30 + S)
    want = Z.oracle_moe(L, x)
    m = gpu_layer(L)
    try:
        check_layer(m, L, x, want)
    finally:
        m.close()


@pytest.mark.parametrize("S", [1, 512])
def test_config4_maple(dev, S, layer_cache):
    """Config 4: Maple shape (MI=768), tq2 experts, clamped SwiGLU."""
    say("config4 maple S", S)
    L = layer_cache("maple", seed=4)
    x = Z.make_input(L, S, 40 + S)
    want = Z.oracle_moe(L, x)
    m = gpu_layer(L)
    try:
        check_layer(m, L, x, want)
    finally:
        m.close()


@pytest.mark.parametrize("S", [1, 4, 8, 64])
def test_ling_grouped_router(dev, S, layer_cache):
    """A13: Ling's grouped router (ling.c:705-789) on the decode (S <= 4), wave-logit
    (S < 16) and exact-logit (S >= 16) paths: ids exact, weights 1e-4, outputs 1e-3."""
    say("ling grouped S", S)
    L = layer_cache("ling", seed=5)
    x = Z.make_input(L, S, 60 + S)
    want = Z.oracle_moe(L, x)
    m = gpu_layer(L)
    try:
        _, _, _, err = check_layer(m, L, x, want)
        say(f"  rel L2 {err:.2e}")
    finally:
        m.close()


def test_config1_gemma_s1_many_tokens(dev, layer_cache):
    """Config 1 at S=1 over 64 independent residuals (routing ids exact on each)."""
    say("config1 gemma S=1 x64")
    L = layer_cache("gemma", seed=1)
    m = gpu_layer(L)
    try:
        for i in range(64):
            x = Z.make_input(L, 1, 100 + i)
            want = Z.oracle_moe(L, x)
            check_layer(m, L, x, want)
    finally:
        m.close()


@pytest.mark.parametrize("kind,kw", [("gemma", dict()), ("lfm", dict()), ("maple", dict(E=64))])
def test_small_batches_both_paths(dev, kind, kw, layer_cache):
    """S = 2, 3, 4, 5 against the oracle: the fused decode kernels take S <= 2 for q4_0 /
    q8_0 weights and S <= 4 for tq2, the matrix-core path the rest, so each format
    crosses from one path to the other inside this range."""
    L = layer_cache(kind, seed=21, **kw)
    m = gpu_layer(L)
    try:
        for S in (2, 3, 4, 5):
            say(f"case {kind} S={S}")
            x = Z.make_input(L, S, 60 + S)
            check_layer(m, L, x, Z.oracle_moe(L, x))
    finally:
        m.close()


# --------------------------------------------------------------- properties
def test_batch_invariance(dev, layer_cache):
    """Tokens do not interact in a MoE layer: one S=96 call equals three S=32 calls
    bit for bit (the engines' --nobatch check, gemma4.c:3191-3197)."""
    L = layer_cache("gemma", seed=2, E=16)
    x = Z.make_input(L, 96, 50)
    m = gpu_layer(L)
    try:
        a, ea, wa = m.forward(x)
        parts = [m.forward(x[i:i + 32]) for i in (0, 32, 64)]
        assert np.array_equal(ea, np.concatenate([p[1] for p in parts]))
        assert np.array_equal(a.view(np.uint32), np.concatenate([p[0] for p in parts]).view(np.uint32))
    finally:
        m.close()


def test_chunked_large_batch(dev, layer_cache):
    """S beyond one dispatch chunk (8192 pairs) is split by the library; results
    equal per-chunk calls."""
    L = layer_cache("lfm", seed=3, E=8, fmts=(1, 1, 1), D=512, MI=256, K=4)
    S = 2048 + 100
    x = Z.make_input(L, S, 51)
    m = gpu_layer(L)
    try:
        a, ea, _ = m.forward(x)
        b1, e1, _ = m.forward(x[:2048])
        b2, e2, _ = m.forward(x[2048:])
        assert np.array_equal(ea, np.concatenate([e1, e2]))
        assert np.array_equal(a.view(np.uint32), np.concatenate([b1, b2]).view(np.uint32))
        want = Z.oracle_moe(L, x)
        assert np.array_equal(ea, want.eidx) and Z.rel_l2(a, want.out) < OUT_TOL
    finally:
        m.close()


def test_begin_end_and_dev_paths(dev, layer_cache):
    import torch
    L = layer_cache("gemma", seed=2, E=16)
    x = Z.make_input(L, 12, 52)
    m = gpu_layer(L)
    try:
        a, ea, wa = m.forward(x)
        lib = zz.lib()
        assert lib.zz_moe_forward_begin(m.id, x.ctypes.data_as(zz._f32p), 12) == 1
        out = np.zeros_like(a)
        e2 = np.zeros_like(ea)
        w2 = np.zeros_like(wa)
        assert lib.zz_moe_forward_end(m.id, out.ctypes.data_as(zz._f32p), e2.ctypes.data_as(zz._i32p),
                                      w2.ctypes.data_as(zz._f32p)) == 1
        assert np.array_equal(out.view(np.uint32), a.view(np.uint32)) and np.array_equal(e2, ea)
        st = torch.cuda.Stream()             # handle 0 would select the library's stream
        with torch.cuda.stream(st):
            dx = torch.from_numpy(x).cuda()
            dy = torch.zeros_like(dx)
            de = torch.zeros(12 * L.K, dtype=torch.int32, device="cuda")
            m.forward_dev(dx.data_ptr(), dy.data_ptr(), 12, de.data_ptr(), 0, st.cuda_stream)
        st.synchronize()
        assert np.array_equal(dy.cpu().numpy().view(np.uint32), a.view(np.uint32))
        assert np.array_equal(de.cpu().numpy(), ea)
    finally:
        m.close()


def test_empty_and_bad_calls_decline(dev, layer_cache):
    """An empty batch, a missing buffer, an unknown layer and an end with nothing begun
    return 0 with a message and launch nothing; the layer then runs as before."""
    L = layer_cache("gemma", seed=2, E=16)
    x = Z.make_input(L, 5, 53)
    m = gpu_layer(L)
    try:
        a, ea, _ = m.forward(x)
        lib = zz.lib()
        out = np.zeros_like(a)
        xp, op = x.ctypes.data_as(zz._f32p), out.ctypes.data_as(zz._f32p)
        assert lib.zz_moe_forward(m.id, xp, op, 0, None, None) == 0 and zz.last_error()
        assert lib.zz_moe_forward(m.id, xp, None, 5, None, None) == 0
        assert lib.zz_moe_forward(m.id + 1000, xp, op, 5, None, None) == 0
        assert lib.zz_moe_forward_dev(m.id, None, None, 0, None, None, None) == 0
        assert lib.zz_moe_forward_end(m.id, op, None, None) == 0
        assert not out.any()
        b, eb, _ = m.forward(x)
        assert np.array_equal(b.view(np.uint32), a.view(np.uint32)) and np.array_equal(eb, ea)
    finally:
        m.close()


def test_declines_until_all_experts_resident(dev, layer_cache):
    L = layer_cache("gemma", seed=2, E=16)
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, None, L.pre_ln, L.post_ln)
    try:
        for e in range(L.E - 1):
            m.upload(e, L.experts[e * L.esz:(e + 1) * L.esz])
        x = Z.make_input(L, 2, 53)
        out = np.full((2, L.D), 9.0, np.float32)
        ok = zz.lib().zz_moe_forward(m.id, x.ctypes.data_as(zz._f32p), out.ctypes.data_as(zz._f32p),
                                     2, None, None)
        assert ok == 0 and np.all(out == 9.0)
        assert "uploaded" in zz.last_error()
        bad = np.zeros(L.esz - 1, np.uint8)
        assert zz.lib().zz_moe_expert_upload(m.id, 0, bad.ctypes.data_as(zz._u8p), bad.nbytes) == 0
    finally:
        m.close()


@pytest.mark.parametrize("fmt", [Z.FMT_Q40, Z.FMT_Q80])
def test_device_quantiser_bit_exact(dev, fmt):
    """zz_quantize equals q40_quant_row / q80_quant_row (through the oracle, pinned to
    the compiled reference), including blocks whose fused x*id+8.5 rounding differs
    from the unfused one, all-zero blocks and sign ties in max|x|."""
    import torch
    rng = np.random.default_rng(61)
    w = (rng.standard_normal(32 * 4096) * 0.02).astype(np.float32)
    w[:32] = 0.0
    w[32:64] = 0.01
    w[64] = -0.05
    w[65] = 0.05                                   # first max-|x| element wins
    want = Z.quant_rows(fmt, w.reshape(1, -1))
    dw = torch.from_numpy(w).cuda()
    out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    zz.quantize_dev(fmt, dw.data_ptr(), out.data_ptr(), w.size)
    torch.cuda.synchronize()
    zz.lib().gpu_init()
    assert np.array_equal(out.cpu().numpy(), want)


def test_null_stream_orders_with_the_default_stream(dev):
    """A NULL stream argument (the library's stream) is ordered after work the caller
    queued on the legacy default stream, and before work queued there afterwards, with
    no synchronisation in between: torch fills a large buffer, the library quantises
    it at once, torch overwrites the buffer at once. The output is the quantisation of
    the first fill (a non-blocking library stream read the buffer before it was
    written, and every FlashHead score came out tied)."""
    import torch
    n = 32 * (1 << 20)
    torch.cuda.synchronize()
    f = torch.empty(n, dtype=torch.float32, device="cuda")
    q = torch.zeros(n // 32 * 18, dtype=torch.uint8, device="cuda")
    for _ in range(3):                              # several rounds, fresh values each
        f.fill_(0.25)
        f.mul_(torch.arange(n, device="cuda", dtype=torch.float32).remainder_(7.0).add_(1.0))
        zz.quantize_dev(zz.GPU_FMT_Q40, f.data_ptr(), q.data_ptr(), n, 0)
        f.fill_(float("nan"))                       # must land after the library read
        torch.cuda.synchronize()
        first = (0.25 * (np.arange(64, dtype=np.float32) % 7 + 1)).astype(np.float32)
        want = Z.quant_rows(Z.FMT_Q40, first.reshape(1, -1))
        got = q[:2 * 18].cpu().numpy()
        assert np.array_equal(got, want)
        tail = q[-18:].cpu().numpy()
        assert np.isfinite(Z.dequant_q40(tail, 1, 32)).all()


def test_profile_sessions_do_not_share_events(dev, layer_cache):
    """zz_moe_profile: records stay readable after switching off, and a new session
    reuses their events only after dropping them. Three sessions in a row, each with
    a batched and a decode forward: every kernel time is positive and their sum stays
    within the host's wall time of the forwards."""
    import time
    L = layer_cache("gemma", 0)
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, None, L.pre_ln, L.post_ln, eps=L.eps)
    try:
        m.upload_all(L.experts)
        xb, x1 = Z.make_input(L, 64, 3), Z.make_input(L, 1, 4)
        for session in range(3):
            zz.profile(True)
            t0 = time.perf_counter()
            m.forward(xb)
            m.forward(x1)
            wall_ms = (time.perf_counter() - t0) * 1e3
            zz.profile(False)
            prof = zz.profile_read()
            say(f"session {session}: " + ", ".join(f"{k} {ms:.3f}/{n}" for k, (ms, n) in prof.items() if n))
            assert prof["ffn_down"][1] == 1 and prof["dec_down"][1] == 1
            assert all(ms > 0 for ms, n in prof.values() if n)
            assert sum(ms for ms, _ in prof.values()) <= wall_ms
    finally:
        m.close()


def _layer_from(L):
    return zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                       L.pes, L.bias, L.pre_ln, L.post_ln, norm_topk=L.norm_topk, use_bias=L.use_bias,
                       eps=L.eps, routed_scaling=L.routed_scaling, clamp=L.clamp, n_group=L.n_group,
                       topk_group=L.topk_group)


def test_container_lfm_per_layer_formats(dev, tmp_path):
    """An LFM-shaped container whose layers have different expert formats, one `eszl`
    line each (lfm25.c:326-331): layer 0 q4_0, layer 1 q8_0. zz_moe_load_experts reads
    each layer's records at its own size and format; a layer whose formats are not the
    line's declines with the reason."""
    say("container lfm eszl")
    L0 = Z.make_layer("lfm", seed=31, D=512, MI=256, E=16, K=4, fmts=(Z.FMT_Q40,) * 3)
    L1 = Z.make_layer("lfm", seed=32, D=512, MI=256, E=16, K=4, fmts=(Z.FMT_Q80,) * 3)
    Z.write_moe_container(str(tmp_path), [L0, L1], per_layer=True)
    for li, L in enumerate((L0, L1)):
        m = _layer_from(L)
        try:
            m.load_experts(str(tmp_path), li)
            x = Z.make_input(L, 6, 40 + li)
            out, eidx, ewt = m.forward(x)
            want = Z.oracle_moe(L, x)
            assert np.array_equal(eidx, want.eidx) and Z.rel_l2(out, want.out) < 1e-3
        finally:
            m.close()
    # the record size matches but the line names another format: a mixed layer (gate/up
    # q4_0, down q8_0) under an eszl line that says q4_0 for all three
    L0b = Z.make_layer("lfm", seed=31, D=512, MI=256, E=16, K=4, fmts=(Z.FMT_Q40, Z.FMT_Q40, Z.FMT_Q80))
    Z.write_moe_container(str(tmp_path / "mixed"), [L0b], per_layer=False)
    with open(tmp_path / "mixed" / "manifest.txt") as f:
        text = f.read()
    g, _, d = L0b.tensor_sizes()
    text = text.replace(f"esz {L0b.esz} {g} {d}\n", f"eszl 0 {L0b.esz} {g} {d} 1\n")
    with open(tmp_path / "mixed" / "manifest.txt", "w") as f:
        f.write(text)
    m = _layer_from(L0b)
    try:
        with pytest.raises(RuntimeError, match="format"):
            m.load_experts(str(tmp_path / "mixed"), 0)
    finally:
        m.close()


def test_container_maple_tq2(dev, tmp_path):
    """A Maple-shaped tq2 container (one `esz` line, maple.c:255-258): the records load
    into the slot table and the layer matches the oracle."""
    say("container maple tq2")
    L = Z.make_layer("maple", seed=33, D=512, MI=256, E=32, K=8)
    Z.write_moe_container(str(tmp_path), [L], per_layer=False)
    m = _layer_from(L)
    try:
        m.load_experts(str(tmp_path), 0)
        for S in (1, 9):
            x = Z.make_input(L, S, 50 + S)
            out, eidx, ewt = m.forward(x)
            want = Z.oracle_moe(L, x)
            assert np.array_equal(eidx, want.eidx) and Z.rel_l2(out, want.out) < 1e-3
    finally:
        m.close()
