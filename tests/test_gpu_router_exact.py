"""GPU: the router's exactness machinery, forced. Each case builds inputs that make
one path run, then checks that the routing equals the oracle's (the reference's
arithmetic) and that the library's counter for that path moved, which shows it ran:

  exact ties       duplicated router rows: equal scores go to the lower expert
                   (gemma4.c:604-607, lfm25.c:656-660, maple.c:588-594, ling.c:748-768),
                   zz_moe_stats()[3]; gemma's bounded logits (S < 16) also replay the
                   serial fp32 chain first, [2];
  near ties        lfm scores one float ulp apart;
  libm boundary    a planted lfm/ling logit where glibc's expf (lfm25.c:654) and a
                   correctly rounded exp put a different expert first;
  rmsnorm replay   gemma inputs whose mean square sits on a float rounding boundary, [0];
  logit replay     lfm/maple/ling router rows whose double sum sits on a float
                   rounding boundary, [1];
and the device expf itself against the host's, bit for bit.
"""
import sys

import numpy as np
import pytest

import zzref as Z
import zunzuncito_amd as zz

pytestmark = pytest.mark.gpu

SMALL = dict(D=512, MI=256, E=16)


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def dev():
    return zz.init()


def gpu_layer(L):
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, L.bias, L.pre_ln, L.post_ln, norm_topk=L.norm_topk,
                    use_bias=L.use_bias, eps=L.eps, routed_scaling=L.routed_scaling,
                    clamp=L.clamp, n_group=L.n_group, topk_group=L.topk_group)
    m.upload_all(L.experts)
    return m


def run(L, x):
    """GPU forward and oracle; returns (gpu out, eidx, ewt), the oracle result and
    the counter deltas of the GPU call."""
    m = gpu_layer(L)
    try:
        s0 = np.array(zz.stats(), np.int64)
        out, eidx, ewt = m.forward(x)
        ds = np.array(zz.stats(), np.int64) - s0
    finally:
        m.close()
    return (out, eidx, ewt), Z.oracle_moe(L, x), ds


def check(L, got, want, exact_weights):
    out, eidx, ewt = got
    assert np.array_equal(eidx, want.eidx), (eidx.reshape(-1, L.K)[:4], want.eidx.reshape(-1, L.K)[:4])
    if exact_weights:
        assert np.array_equal(ewt.view(np.uint32), want.ewt.view(np.uint32))
    else:
        np.testing.assert_allclose(ewt, want.ewt, rtol=1e-4, atol=1e-6)
    assert Z.rel_l2(out, want.out) < 1e-3


def small_layer(kind, K=2, seed=3):
    L = Z.make_layer(kind, seed=seed, K=K, **SMALL)
    L.router = (L.router * np.float32(0.01)).astype(np.float32)
    if kind == "ling":
        L.n_group, L.topk_group = 4, 2
    return L


def tie_input(L, S, seed):
    x = Z.make_input(L, S, seed)
    x[:, 0] = 8.0
    return x


# ------------------------------------------------------------------- ties
@pytest.mark.parametrize("kind", ["gemma", "lfm", "maple", "ling"])
@pytest.mark.parametrize("S", [1, 8, 64])
def test_exact_ties_go_to_the_lower_expert(dev, kind, S):
    """Experts with identical router rows (and equal biases) tie exactly, above all
    others; with K = 2 the tie straddles the k-th place. Ling: three groups of two
    tied experts tie as groups too, with two groups kept."""
    say(f"ties {kind} S={S}")
    L = small_layer(kind)
    dup = [4, 5, 8, 9, 12, 13] if kind == "ling" else [3, 6, 11]
    for e in dup:
        L.router[e] = 0.0
        L.router[e, 0] = 4.0
        if L.bias is not None:
            L.bias[e] = 0.0
    x = tie_input(L, S, 70 + S)
    got, want, ds = run(L, x)
    say(f"  counters {ds.tolist()}  first ids {got[1][:L.K].tolist()}")
    assert want.eidx.reshape(S, L.K)[:, 0].tolist() == [dup[0]] * S      # the planted tie is real
    check(L, got, want, exact_weights=kind != "gemma" or S >= 16)
    assert ds[3] == S                                   # every token met the tie
    if kind == "gemma" and S < 16:
        assert ds[2] == S                               # bounded logits: replayed first


@pytest.mark.parametrize("S", [1, 8, 64])
def test_lfm_scores_one_ulp_apart(dev, S):
    """Saturated sigmoid scores 1.0 plus biases 0 and 2^-23: one float ulp apart, the
    higher one first, then a tie at the k-th place decided by index."""
    L = small_layer("lfm")
    for e in (3, 6, 11):
        L.router[e] = 0.0
        L.router[e, 0] = 4.0
        L.bias[e] = 0.0
    L.bias[6] = np.float32(2.0 ** -23)
    x = tie_input(L, S, 80 + S)
    got, want, ds = run(L, x)
    assert want.eidx.reshape(S, L.K).tolist() == [[6, 3]] * S
    check(L, got, want, exact_weights=True)
    assert ds[3] == S


# ----------------------------------------------------------- libm boundary
def _glibc_expf(v):
    v = np.ascontiguousarray(v, np.float32)
    y = np.zeros_like(v)
    Z.oracle().orc_expf(Z.ptr(v), Z.ptr(y), v.size)
    return y


def _plant_expf_case():
    """(xa, xb, bias_b): sigmoid scores s(-xa) by glibc and by a correctly rounded
    exp differ, and s(-xb) + bias_b lands strictly between them."""
    xa = np.float32(float.fromhex("0x1.00001cp+1"))
    ea = _glibc_expf(np.array([xa]))[0]
    ea_cr = np.float32(np.exp(np.float64(xa)))
    sa = np.float32(1) / (np.float32(1) + ea)
    sa_cr = np.float32(1) / (np.float32(1) + ea_cr)
    assert sa != sa_cr
    mid = np.nextafter(min(sa, sa_cr), np.float32(1))
    assert min(sa, sa_cr) < mid < max(sa, sa_cr)
    for k in range(1, 200):                         # a nearby logit where the two agree
        xb = np.float32(xa + np.float32(k) * np.spacing(xa))
        eb = _glibc_expf(np.array([xb]))[0]
        if eb != np.float32(np.exp(np.float64(xb))):
            continue
        sb = np.float32(1) / (np.float32(1) + eb)
        bias = np.float32(mid - sb)
        if np.float32(sb + bias) == mid:
            return xa, xb, bias, sa, sa_cr, mid
    raise AssertionError("no companion logit found")


@pytest.mark.parametrize("kind", ["lfm", "ling"])
@pytest.mark.parametrize("S", [1, 8, 64])
def test_selection_decided_by_glibc_expf(dev, kind, S):
    """Expert 2's logit is -xa exactly, expert 1's is -xb plus a bias that puts its
    score strictly between expert 2's score under glibc's expf and under a correctly
    rounded exp, so the two exps choose different experts for the single slot."""
    xa, xb, bias_b, sa, sa_cr, mid = _plant_expf_case()
    L = Z.make_layer(kind, seed=4, K=1, **SMALL)
    if kind == "ling":
        L.n_group, L.topk_group = 1, 1
    L.router[:] = 0.0
    L.router[2, 1] = -1.0
    L.router[1, 2] = -1.0
    L.bias[:] = -1.0
    L.bias[2] = 0.0
    L.bias[1] = bias_b
    x = Z.make_input(L, S, 90 + S)
    x[:, 1] = xa
    x[:, 2] = xb
    got, want, _ = run(L, x)
    ref_first = 1 if mid > sa else 2
    cr_first = 1 if mid > sa_cr else 2
    say(f"  {kind} S={S}: glibc picks {ref_first}, a correctly rounded exp would pick {cr_first}")
    assert ref_first != cr_first
    assert want.eidx.tolist() == [ref_first] * S
    check(L, got, want, exact_weights=True)


def test_router_expf_matches_host_expf(dev):
    """zz_router_expf (the device expf of the sigmoid routers) against the host's
    glibc expf: every 251st 32-bit pattern, the overflow and underflow thresholds
    and their neighbours, and the subnormal-result range densely."""
    import torch
    pats = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x42b17217, 0x42b17218, 0xc2cff1b4, 0xc2cff1b5, 0xc2ce8ed0, 0xff800000,
                      0x7f800000, 0x7fc00000, 0x00000000, 0x80000000, 0x42b00000, 0xc2b00000], np.uint32)
    sub = np.arange(0xc2ae0000, 0xc2d00000, 3, dtype=np.uint32)      # about -87 .. -104
    x = np.concatenate([pats, edges, sub]).view(np.float32)
    want = _glibc_expf(x)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty_like(dx)
    assert zz.lib().zz_router_expf(dx.data_ptr(), dy.data_ptr(), x.size, None) == 1, zz.last_error()
    torch.cuda.synchronize()
    got = dy.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    bad = np.nonzero(got[~nan].view(np.uint32) != want[~nan].view(np.uint32))[0]
    say(f"  {x.size} inputs, {bad.size} differ")
    assert bad.size == 0, (x[~nan][bad[:4]], got[~nan][bad[:4]], want[~nan][bad[:4]])


# ----------------------------------------------------------------- replays
def _rms_boundary_row(D, rng):
    """A row whose sum of squares is within 1e-12 of D * (1 + 2^-24), so that its mean
    square sits on the float rounding boundary between 1 and 1 + 2^-23."""
    target = D * (1.0 + 2.0 ** -24)
    rest = float(D - 2)
    a = np.float32(np.sqrt(target - rest))
    while float(a) ** 2 > target - rest:
        a = np.nextafter(a, np.float32(0))
    b = np.float32(np.sqrt(target - rest - float(a) ** 2))
    row = np.ones(D, np.float32)
    row[rng.permutation(D)[:2]] = [a, b]
    assert abs(float(np.sum(row.astype(np.float64) ** 2)) - target) < 1e-9
    return row


@pytest.mark.parametrize("S", [1, 8])
def test_gemma_rmsnorm_serial_replay(dev, S):
    say(f"rmsnorm replay S={S}")
    L = Z.make_layer("gemma", seed=6, K=4, **SMALL)
    rng = np.random.default_rng(S)
    x = np.stack([_rms_boundary_row(L.D, rng) for _ in range(S)])
    got, want, ds = run(L, x)
    say(f"  counters {ds.tolist()}")
    check(L, got, want, exact_weights=False)
    assert ds[0] >= S


@pytest.mark.parametrize("kind", ["lfm", "maple", "ling"])
@pytest.mark.parametrize("S", [1, 8])
def test_logit_serial_replay(dev, kind, S):
    """Expert 5's logit is 1 + 2^-24 (+ 2^-60, lost in the serial double sum): a
    float rounding tie that no certified parallel sum can settle; expert 7's is
    1 + 2^-23, the value a correctly rounded sum would give expert 5."""
    say(f"logit replay {kind} S={S}")
    L = Z.make_layer(kind, seed=7, K=2, **SMALL)
    if kind == "ling":
        L.n_group, L.topk_group = 4, 2
    L.router = (L.router * np.float32(0.01)).astype(np.float32)
    L.router[5] = 0.0
    L.router[5, :3] = [1.0, 2.0 ** -24, 2.0 ** -60]
    L.router[7] = 0.0
    L.router[7, :2] = [1.0, 2.0 ** -23]
    if L.bias is not None:
        L.bias[5] = L.bias[7] = 0.0
    x = Z.make_input(L, S, 95 + S)
    x[:, :3] = 1.0
    got, want, ds = run(L, x)
    say(f"  counters {ds.tolist()}  ids {got[1][:L.K].tolist()}")
    check(L, got, want, exact_weights=True)
    assert ds[1] >= S


# ------------------------------------------------------- certified double logits
def _cancelling_layer(kind, seed):
    """Router rows whose dot with the input nearly cancels: two large equal and
    opposite terms dwarf the rest, so the exact-order prefix sums are large against
    the logit and many logits sit near a float rounding boundary of their bound."""
    L = small_layer(kind, seed=seed)
    rng = np.random.default_rng(seed)
    L.router[:, 3] = (rng.standard_normal(L.E) * 300).astype(np.float32)
    L.router[:, 7] = -L.router[:, 3]
    return L


@pytest.mark.parametrize("kind", ["lfm", "maple", "ling"])
@pytest.mark.parametrize("S", [1, 3, 5, 8, 15])
@pytest.mark.parametrize("cancel", [False, True])
def test_certified_double_logits(dev, kind, S, cancel):
    """Below S = 16 the lfm / maple / ling logits come from the wave-parallel sum with
    the prefix-sum bound of the reference's serial double chain (and a replay where
    the bound spans a float rounding boundary): they equal the reference's floats bit
    for bit, and the routing follows."""
    L = _cancelling_layer(kind, 11 + S) if cancel else small_layer(kind, seed=11 + S)
    x = Z.make_input(L, S, 40 + S)
    if cancel:
        x[:, 3] = x[:, 7] = 1.0
    m = gpu_layer(L)
    try:
        s0 = np.array(zz.stats(), np.int64)
        out, eidx, ewt = m.forward(x)
        ds = np.array(zz.stats(), np.int64) - s0
        got = m.debug(S, logits=True)["logits"]
    finally:
        m.close()
    want = Z.oracle_moe(L, x, dump=True)
    say(f"  {kind} S={S} cancel={cancel}: logit replays {ds[1]}")
    bad = got.astype(np.float32).view(np.uint32) != want.dump["logits"].view(np.uint32)
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:4])
    check(L, (out, eidx, ewt), want, exact_weights=True)
