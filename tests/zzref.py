"""Test-side helpers: ctypes bindings to the CPU oracle (oracle/liboracle.so), to
the compiled reference (oracle/_ref/libref_*.so, present only where it was built),
and seeded synthetic layers shaped like the BASELINE configs.

Test infrastructure only; the product package never imports this module.
"""
import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")

FMT_Q40, FMT_Q80, FMT_TQ2, FMT_Q4A = 1, 2, 3, 4
GATE_GEMMA, GATE_LFM, GATE_MAPLE, GATE_LING = 0, 1, 2, 4   # the library's ZZ_GATE_* codes
ACT_GEGLU_TANH, ACT_SWIGLU, ACT_SWIGLU_CL = 0, 1, 2

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)
u8p = C.POINTER(C.c_uint8)
i8p = C.POINTER(C.c_int8)


def ptr(a, t=None):
    """ctypes pointer to a contiguous numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    if t is None:
        t = {np.float32: f32p, np.int32: i32p, np.uint8: u8p, np.int8: i8p}[a.dtype.type]
    return a.ctypes.data_as(t)


class OrcCfg(C.Structure):
    _fields_ = [("D", C.c_int), ("MI", C.c_int), ("E", C.c_int), ("K", C.c_int),
                ("gating", C.c_int), ("act", C.c_int),
                ("fmt_gate", C.c_int), ("fmt_up", C.c_int), ("fmt_down", C.c_int),
                ("norm_topk", C.c_int), ("use_bias", C.c_int),
                ("eps", C.c_float), ("routed_scaling", C.c_float), ("clamp", C.c_float),
                ("n_group", C.c_int), ("topk_group", C.c_int)]


class OrcWeights(C.Structure):
    _fields_ = [("router", f32p), ("router_scale", f32p), ("pes", f32p), ("bias", f32p),
                ("pre_ln", f32p), ("post_ln", f32p), ("experts", u8p), ("esz", C.c_int64)]


class OrcDump(C.Structure):
    _fields_ = [("xin", f32p), ("xq", i8p), ("xs", f32p), ("xtot", f32p),
                ("hq", i8p), ("hs", f32p), ("htot", f32p), ("logits", f32p)]


_oracle = None


def oracle():
    """The restatement library; built by `make -C oracle` (or __graft_entry__.build)."""
    global _oracle
    if _oracle is None:
        path = os.path.join(ORACLE_DIR, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        L.orc_h2f.restype = C.c_float
        L.orc_h2f.argtypes = [C.c_uint16]
        L.orc_f2h.restype = C.c_uint16
        L.orc_f2h.argtypes = [C.c_float]
        for n in ("orc_q40_dot", "orc_q80_dot"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [u8p, i8p, f32p, C.c_int]
        L.orc_tq2_dot.restype = C.c_float
        L.orc_tq2_dot.argtypes = [u8p, C.c_float, i8p, f32p, C.c_float, C.c_int]
        L.orc_tq2_quant_act.restype = C.c_float
        L.orc_tq2_quant_act.argtypes = [f32p, i8p, f32p, C.c_int]
        L.orc_quant_act.argtypes = [f32p, i8p, f32p, C.c_int]
        for n in ("orc_q40_dot_f32", "orc_q80_dot_f32"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [u8p, f32p, C.c_int]
        L.orc_tq2_dot_f32.restype = C.c_float
        L.orc_tq2_dot_f32.argtypes = [u8p, C.c_float, f32p, C.c_int]
        L.orc_q4a_dot_f32.restype = C.c_float
        L.orc_q4a_dot_f32.argtypes = [u8p, f32p, C.c_int]
        L.orc_tensor_bytes.restype = C.c_int64
        L.orc_tensor_bytes.argtypes = [C.c_int, C.c_int, C.c_int]
        L.orc_moe_layer.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), f32p, C.c_int,
                                    f32p, i32p, f32p, i32p, i32p, C.POINTER(OrcDump)]
        L.orc_route.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), f32p, i32p, f32p, f32p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_expf.argtypes = [f32p, f32p, C.c_longlong]
        L.orc_blockdots.argtypes = [C.c_int, u8p, i8p, C.c_int, i32p]
        L.orc_matmul_f32.argtypes = [C.c_int, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int]
        L.orc_dispatch.argtypes = [i32p, f32p, C.c_int, C.c_int, i32p, C.c_int, i32p, i32p,
                                   f32p, i32p]
        L.orc_set_plant.argtypes = [C.c_int]
        _oracle = L
    return _oracle


def ref_lib(name):
    """A compiled-reference library, or None where oracle/_ref was not built."""
    path = os.path.join(ORACLE_DIR, "_ref", f"libref_{name}.so")
    if not os.path.exists(path):
        return None
    return C.CDLL(path)


# ---------------------------------------------------------------- quantisers
def quant_rows(fmt, w):
    """Quantise an f32 [O, I] matrix with the oracle's reference-exact quantisers."""
    L = oracle()
    w = np.ascontiguousarray(w, dtype=np.float32)
    O, I = w.shape
    if fmt == FMT_Q40:
        rb = I // 32 * 18
        fn = L.orc_q40_quant_row
    elif fmt == FMT_Q80:
        rb = I // 32 * 34
        fn = L.orc_q80_quant_row
    else:
        raise ValueError(fmt)
    out = np.empty(O * rb, dtype=np.uint8)
    fn.argtypes = [f32p, u8p, C.c_int]
    fn(ptr(w.reshape(-1)), ptr(out), O * I)      # blocks are independent: one call
    return out


def tq2_tensor(codes, alpha):
    """tq2 tensor bytes (alpha[O] f32, then packed code rows) from codes[O, I] in {0,1,2}."""
    L = oracle()
    O, I = codes.shape
    L.orc_tq2_pack_row.argtypes = [i8p, u8p, C.c_int]
    packed = np.empty(O * (I // 4), dtype=np.uint8)
    c8 = np.ascontiguousarray(codes, dtype=np.int8).reshape(-1)
    L.orc_tq2_pack_row(ptr(c8), ptr(packed), O * I)   # 64-groups are independent
    return np.concatenate([np.ascontiguousarray(alpha, np.float32).view(np.uint8), packed])


def tensor_bytes(fmt, O, I):
    if fmt == FMT_Q40:
        return O * (I // 32) * 18
    if fmt == FMT_Q80:
        return O * (I // 32) * 34
    if fmt == FMT_Q4A:
        return O * (I // 64) * 36
    return O * 4 + O * (I // 4)


def q4a_rows(rng, O, I, specials=False):
    """Random Q4A rows (tq2.h:269-292): per 64-group an fp16 scale d > 0 and an fp16
    bias m of either sign (the ranges of maple.c:1790-1796), then random nibbles.
    With specials, some groups' d or m is NaN, +-inf, -0 or subnormal."""
    W = rng.integers(0, 256, size=(O * (I // 64), 36), dtype=np.uint8)
    d = (0.002 + 0.01 * np.abs(rng.standard_normal(W.shape[0]))).astype(np.float16)
    m = (0.05 * rng.standard_normal(W.shape[0])).astype(np.float16)
    W[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    W[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    if specials:
        pick = rng.choice(W.shape[0], size=min(12, W.shape[0]), replace=False)
        for k, g in enumerate(pick):
            h = [0x7e00, 0x7c00, 0xfc00, 0x8000, 0x0001, 0x03ff][k % 6]
            off = 0 if k % 2 == 0 else 2
            W[g, off], W[g, off + 1] = h & 255, h >> 8
    return W.reshape(-1)


# ------------------------------------------------------------ synthetic layers
@dataclass
class Layer:
    """A seeded MoE layer in the reference's record layout ([gate | up | down])."""
    D: int
    MI: int
    E: int
    K: int
    gating: int
    act: int
    fmts: tuple
    norm_topk: int = 1
    use_bias: int = 0
    eps: float = 1e-6
    routed_scaling: float = 1.0
    clamp: float = 7.0
    n_group: int = 1
    topk_group: int = 1
    router: np.ndarray = None
    router_scale: np.ndarray = None
    pes: np.ndarray = None
    bias: np.ndarray = None
    pre_ln: np.ndarray = None
    post_ln: np.ndarray = None
    experts: np.ndarray = None
    esz: int = 0
    seed: int = 0
    _keep: list = field(default_factory=list)

    def cfg(self):
        return OrcCfg(self.D, self.MI, self.E, self.K, self.gating, self.act,
                      self.fmts[0], self.fmts[1], self.fmts[2], self.norm_topk, self.use_bias,
                      self.eps, self.routed_scaling, self.clamp, self.n_group, self.topk_group)

    def weights(self):
        return OrcWeights(ptr(self.router), ptr(self.router_scale), ptr(self.pes),
                          ptr(self.bias), ptr(self.pre_ln), ptr(self.post_ln),
                          ptr(self.experts), self.esz)

    def tensor_sizes(self):
        g = tensor_bytes(self.fmts[0], self.MI, self.D)
        u = tensor_bytes(self.fmts[1], self.MI, self.D)
        d = tensor_bytes(self.fmts[2], self.D, self.MI)
        return g, u, d


def _normal(rng, shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def make_expert_q(rng, fmt, O, I, sigma=0.02):
    return quant_rows(fmt, _normal(rng, (O, I), sigma))


_TQ2_LUT = np.array([1] * 102 + [0] * 77 + [2] * 77, dtype=np.int8)


def make_expert_tq2(rng, O, I, sigma=0.02):
    """Ternary codes with P(weight 0) = 102/256 ~ 0.4 and P(+1) = P(-1) = 77/256,
    one f32 alpha per row (tq2.h:17-28): alpha ~ the absmean of an N(0, sigma)
    row, sigma*sqrt(2/pi), with 5% per-row jitter."""
    u = rng.integers(0, 256, size=O * I, dtype=np.uint8)
    codes = _TQ2_LUT[u].reshape(O, I)
    alpha = (sigma * np.sqrt(2 / np.pi) * (1 + 0.05 * rng.standard_normal(O))).astype(np.float32)
    return tq2_tensor(codes, alpha)


def make_layer(kind, seed=1, E=None, D=None, MI=None, K=None, zipf=False, fmts=None):
    """Seeded layer shaped like a BASELINE config.

    kind: "gemma" (config 1/2), "lfm" (config 3: gate/up q4_0, down q8_0 unless
    fmts is given), "maple" (config 4: tq2)."""
    rng = np.random.default_rng(seed)
    if kind == "gemma":
        D, MI, E, K = D or 2816, MI or 704, E or 128, K or 8
        L = Layer(D, MI, E, K, GATE_GEMMA, ACT_GEGLU_TANH, fmts or (FMT_Q40,) * 3, eps=1e-6)
        L.router = _normal(rng, (E, D))
        L.router_scale = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        L.pes = (1 + 0.1 * rng.random(E)).astype(np.float32)
        L.pre_ln = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        L.post_ln = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        if zipf:
            rank = rng.permutation(E) + 1
            L.bias = (-1.1 * np.log(rank)).astype(np.float32)
            L.use_bias = 1
    elif kind == "lfm":
        D, MI, E, K = D or 2048, MI or 1792, E or 32, K or 4
        L = Layer(D, MI, E, K, GATE_LFM, ACT_SWIGLU, fmts or (FMT_Q40, FMT_Q40, FMT_Q80),
                  norm_topk=1, use_bias=1, routed_scaling=1.0)
        L.router = _normal(rng, (E, D))
        L.bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
    elif kind == "ling":
        # Ling-3.0-tiny's router (ling.c:705-789): 128 experts in 8 groups, the best 4
        # groups, top-8; SwiGLU experts of one format per layer
        D, MI, E, K = D or 2048, MI or 512, E or 128, K or 8
        L = Layer(D, MI, E, K, GATE_LING, ACT_SWIGLU, fmts or (FMT_Q40,) * 3, norm_topk=1,
                  use_bias=1, routed_scaling=2.5, n_group=8 if E % 8 == 0 else 1,
                  topk_group=4 if E % 8 == 0 else 1)
        L.router = _normal(rng, (E, D), 0.05)
        L.bias = (0.05 * rng.standard_normal(E)).astype(np.float32)
    elif kind == "maple":
        D, MI, E, K = D or 2048, MI or 768, E or 256, K or 8
        L = Layer(D, MI, E, K, GATE_MAPLE, ACT_SWIGLU_CL, (FMT_TQ2,) * 3, norm_topk=1, clamp=7.0)
        L.router = _normal(rng, (E, D))
    else:
        raise ValueError(kind)
    L.seed = seed
    g, u, d = L.tensor_sizes()
    L.esz = g + u + d
    L.experts = np.empty(E * L.esz, dtype=np.uint8)
    for e in range(E):
        rec = L.experts[e * L.esz:(e + 1) * L.esz]
        parts = []
        for fmt, (O, I) in zip(L.fmts, ((MI, D), (MI, D), (D, MI))):
            if fmt == FMT_TQ2:
                parts.append(make_expert_tq2(rng, O, I))
            else:
                parts.append(make_expert_q(rng, fmt, O, I))
        rec[:] = np.concatenate(parts)
    return L


def make_input(L, S, seed):
    rng = np.random.default_rng(10_000 + seed)
    return _normal(rng, (S, L.D))


# --------------------------------------------------------------- layer calls
@dataclass
class MoeResult:
    out: np.ndarray
    eidx: np.ndarray
    ewt: np.ndarray
    uniq: np.ndarray
    dump: dict = None


def oracle_moe(L, x, dump=False):
    S = x.shape[0]
    out = np.zeros((S, L.D), np.float32)
    eidx = np.zeros(S * L.K, np.int32)
    ewt = np.zeros(S * L.K, np.float32)
    uniq = np.zeros(L.E, np.int32)
    nu = C.c_int(0)
    d = None
    dp = None
    if dump:
        d = dict(xin=np.zeros((S, L.D), np.float32), xq=np.zeros((S, L.D), np.int8),
                 xs=np.zeros((S, L.D // 32), np.float32), xtot=np.zeros(S, np.float32),
                 hq=np.zeros((S * L.K, L.MI), np.int8),
                 hs=np.zeros((S * L.K, L.MI // 32), np.float32),
                 htot=np.zeros(S * L.K, np.float32), logits=np.zeros((S, L.E), np.float32))
        dp = C.byref(OrcDump(*(ptr(d[k]) for k in ("xin", "xq", "xs", "xtot", "hq", "hs", "htot", "logits"))))
    cfg, w = L.cfg(), L.weights()
    rc = oracle().orc_moe_layer(C.byref(cfg), C.byref(w), ptr(np.ascontiguousarray(x, np.float32)),
                                S, ptr(out), ptr(eidx), ptr(ewt), ptr(uniq), C.byref(nu), dp)
    assert rc == 0
    return MoeResult(out, eidx, ewt, uniq[:nu.value].copy(), d)


def ref_moe(L, x):
    """The compiled reference, or None where it is unavailable or cannot express L."""
    S = x.shape[0]
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros((S, L.D), np.float32)
    eidx = np.zeros(S * L.K, np.int32)
    ewt = np.zeros(S * L.K, np.float32)
    uniq = np.zeros(L.E, np.int32)
    nu = C.c_int(0)
    if L.gating == GATE_GEMMA:
        lib = ref_lib("gemma4")
        if lib is None or L.use_bias or L.fmts != (FMT_Q40,) * 3:
            return None
        xin = np.zeros((S, L.D), np.float32)
        rc = lib.ref_g4_moe(L.D, L.MI, L.E, L.K, C.c_float(L.eps), ptr(L.router),
                            ptr(L.router_scale), ptr(L.pes), ptr(L.pre_ln), ptr(L.post_ln),
                            ptr(L.experts), C.c_int64(L.esz), ptr(x), S, ptr(out), ptr(eidx),
                            ptr(ewt), ptr(uniq), C.byref(nu), ptr(xin))
    elif L.gating == GATE_LFM:
        lib = ref_lib("lfm25")
        if lib is None or len(set(L.fmts)) != 1:
            return None
        rc = lib.ref_lfm_moe(L.D, L.MI, L.E, L.K, L.fmts[0], L.norm_topk, L.use_bias,
                             C.c_float(L.routed_scaling), ptr(L.router), ptr(L.bias),
                             ptr(L.experts), C.c_int64(L.esz), ptr(x), S, ptr(out), ptr(eidx),
                             ptr(ewt), ptr(uniq), C.byref(nu))
    elif L.gating == GATE_LING:
        lib = ref_lib("ling")
        if lib is None or len(set(L.fmts)) != 1:
            return None
        rc = lib.ref_ling_moe(L.D, L.MI, L.E, L.K, L.fmts[0], L.n_group, L.topk_group, L.norm_topk,
                              C.c_float(L.routed_scaling), ptr(L.router), ptr(L.bias),
                              ptr(L.experts), C.c_int64(L.esz), ptr(x), S, ptr(out), ptr(eidx),
                              ptr(ewt), ptr(uniq), C.byref(nu))
    else:
        lib = ref_lib("maple")
        if lib is None:
            return None
        rc = lib.ref_maple_moe(L.D, L.MI, L.E, L.K, L.norm_topk, C.c_float(L.clamp),
                               ptr(L.router), ptr(L.experts), C.c_int64(L.esz), ptr(x), S,
                               ptr(out), ptr(eidx), ptr(ewt), ptr(uniq), C.byref(nu))
    assert rc == 0
    return MoeResult(out, eidx, ewt, uniq[:nu.value].copy())


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_items(d, tch=64):
    """The FFN work items of a debug dump cover each union entry's pairs exactly:
    the entry's items (expert uniq[u], at most tch pairs each) tile its list
    [offs[u], offs[u+1]) in order without gaps or overlaps. Returns, per union
    entry, the set of XCDs (slot % 8) its items run on."""
    items, uniq, offs = d["items"], d["uniq"], d["offs"]
    assert len(items) % 8 == 0 and len(items) > 0
    xcds = {}
    spans = {}
    for slot, (e, u, p0, n) in enumerate(items):
        if n == 0:
            continue
        assert 0 < n <= tch and 0 <= u < len(uniq) and e == uniq[u], (slot, e, u, n)
        spans.setdefault(u, []).append((p0, n))
        xcds.setdefault(u, set()).add(slot % 8)
    assert sorted(spans) == list(range(len(uniq)))
    for u, sp in spans.items():
        sp.sort()
        assert sum(n for _, n in sp) == offs[u + 1] - offs[u]
        for (a, na), (b, _) in zip(sp, sp[1:]):
            assert b == a + na
    return xcds


# ------------------------------------------- gemma around the MoE block
class OrcDense(C.Structure):
    _fields_ = [("DI", C.c_int), ("mlp", u8p), ("pre_ffn_ln", f32p), ("post_ffn_ln1", f32p),
                ("post_ffn_ln", f32p), ("layer_scalar", C.c_float)]


@dataclass
class Dense:
    """gemma's dense MLP branch and layer combine weights (gemma4.c:1003-1030)."""
    D: int
    DI: int
    mlp: np.ndarray            # q4_0 mlp_gate [DI,D] | mlp_up [DI,D] | mlp_down [D,DI]
    pre_ffn_ln: np.ndarray
    post_ffn_ln1: np.ndarray
    post_ffn_ln: np.ndarray
    layer_scalar: float

    def orc(self):
        return OrcDense(self.DI, ptr(self.mlp), ptr(self.pre_ffn_ln), ptr(self.post_ffn_ln1),
                        ptr(self.post_ffn_ln), self.layer_scalar)


def make_dense(D, DI, seed):
    rng = np.random.default_rng(20_000 + seed)
    mlp = np.concatenate([make_expert_q(rng, FMT_Q40, DI, D), make_expert_q(rng, FMT_Q40, DI, D),
                          make_expert_q(rng, FMT_Q40, D, DI)])
    ln = lambda: (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)   # noqa: E731
    return Dense(D, DI, mlp, ln(), ln(), ln(), float(np.float32(0.5 + rng.random())))


def make_table(V, D, seed):
    """A seeded tied q4_0 embedding / lm_head [V, D] and its final norm."""
    rng = np.random.default_rng(30_000 + seed)
    table = make_expert_q(rng, FMT_Q40, V, D, sigma=0.05)
    fnorm = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    return table, fnorm


def _bind_gemma(L):
    L.orc_dense_mlp.argtypes = [C.POINTER(OrcDense), C.c_int, C.c_float, f32p, C.c_int, f32p]
    L.orc_gemma_ffn_block.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.POINTER(OrcDense),
                                      f32p, C.c_int, i32p, f32p]
    L.orc_embed_row.argtypes = [u8p, C.c_int, C.c_float, C.c_int, f32p]
    L.orc_head.argtypes = [u8p, C.c_int, C.c_int, f32p, C.c_float, C.c_float, f32p, f32p]
    return L


def oracle_dense(dn, eps, H):
    L = _bind_gemma(oracle())
    H = np.ascontiguousarray(H, np.float32)
    out = np.zeros_like(H)
    o = dn.orc()
    L.orc_dense_mlp(C.byref(o), dn.D, C.c_float(eps), ptr(H), H.shape[0], ptr(out))
    return out


def oracle_block(L_, dn, H):
    """(H', eidx, ewt) of orc_gemma_ffn_block."""
    L = _bind_gemma(oracle())
    H = np.array(H, np.float32, order="C", copy=True)
    S = H.shape[0]
    eidx = np.zeros(S * L_.K, np.int32)
    ewt = np.zeros(S * L_.K, np.float32)
    cfg, w, o = L_.cfg(), L_.weights(), dn.orc()
    assert L.orc_gemma_ffn_block(C.byref(cfg), C.byref(w), C.byref(o), ptr(H), S, ptr(eidx), ptr(ewt)) == 0
    return H, eidx, ewt


def ref_block(L_, dn, H):
    """The compiled reference's FFN half of layer_fwd, or None where unavailable."""
    lib = ref_lib("gemma4")
    if lib is None or L_.use_bias or L_.fmts != (FMT_Q40,) * 3:
        return None
    H = np.array(H, np.float32, order="C", copy=True)
    S = H.shape[0]
    eidx = np.zeros(S * L_.K, np.int32)
    ewt = np.zeros(S * L_.K, np.float32)
    rc = lib.ref_g4_ffn_block(L_.D, L_.MI, L_.E, L_.K, dn.DI, C.c_float(L_.eps), ptr(L_.router),
                              ptr(L_.router_scale), ptr(L_.pes), ptr(L_.pre_ln), ptr(L_.post_ln),
                              ptr(L_.experts), C.c_int64(L_.esz), ptr(dn.mlp), ptr(dn.pre_ffn_ln),
                              ptr(dn.post_ffn_ln1), ptr(dn.post_ffn_ln), C.c_float(dn.layer_scalar),
                              ptr(H), S, ptr(eidx), ptr(ewt))
    assert rc == 0
    return H, eidx, ewt


def oracle_embed(table, D, scale, toks):
    L = _bind_gemma(oracle())
    out = np.zeros((len(toks), D), np.float32)
    for i, t in enumerate(toks):
        L.orc_embed_row(ptr(table), D, C.c_float(scale), int(t), ptr(out[i]))
    return out


def ref_embed(table, V, D, scale, toks):
    lib = ref_lib("gemma4")
    if lib is None:
        return None
    lib.ref_g4_embed.argtypes = [u8p, C.c_int, C.c_int, C.c_float, C.c_int, f32p]
    out = np.zeros((len(toks), D), np.float32)
    for i, t in enumerate(toks):
        lib.ref_g4_embed(ptr(table), V, D, C.c_float(scale), int(t), ptr(out[i]))
    return out


def oracle_head(table, V, D, fnorm, eps, cap, H):
    L = _bind_gemma(oracle())
    H = np.ascontiguousarray(H, np.float32)
    lg = np.zeros((H.shape[0], V), np.float32)
    am = np.array([L.orc_head(ptr(table), V, D, ptr(fnorm), C.c_float(eps), C.c_float(cap),
                              ptr(H[s]), ptr(lg[s])) for s in range(H.shape[0])], np.int32)
    return lg, am


def ref_head(table, V, D, fnorm, eps, cap, H):
    lib = ref_lib("gemma4")
    if lib is None:
        return None
    lib.ref_g4_head.argtypes = [u8p, C.c_int, C.c_int, f32p, C.c_float, C.c_float, f32p, f32p]
    H = np.ascontiguousarray(H, np.float32)
    lg = np.zeros((H.shape[0], V), np.float32)
    am = np.array([lib.ref_g4_head(ptr(table), V, D, ptr(fnorm), C.c_float(eps), C.c_float(cap),
                                   ptr(H[s]), ptr(lg[s])) for s in range(H.shape[0])], np.int32)
    return lg, am


def dequant_q40(table, V, D):
    """f32 [V, D] of a q4_0 [V, D] table (q40.h:9-18: fp16 d, then 16 bytes of
    nibbles, low = weights 0..15, high = 16..31, value d * (q - 8))."""
    b = np.frombuffer(np.ascontiguousarray(table), np.uint8).reshape(V, D // 32, 18)
    d = b[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    q = b[:, :, 2:]
    w = np.concatenate([(q & 15), (q >> 4)], axis=2).astype(np.float32) - 8.0
    return (w * d[:, :, None]).reshape(V, D)


@dataclass
class Flash:
    """A FlashHead for a tied table (tools/flashhead.py's tensors): q4_0 centroids
    [NC, D], token_map [NC, CS] (-1 = padding), cluster_scale [NC], force ids."""
    cent: np.ndarray
    NC: int
    tmap: np.ndarray
    CS: int
    NP: int
    cscale: np.ndarray
    scaled: int
    force: np.ndarray

    @property
    def nforce(self):
        return int(self.force.size)


def make_flash(table, V, D, NC, CS, NP, nforce=3, seed=0, scaled=1, tie_all=False):
    """A balanced clustering of the table's rows: a seeded permutation of the V ids in
    NC rows of CS (NC * CS - V padding slots of -1 spread over them), each centroid the members' mean direction
    times the largest member norm (the scale folded in when `scaled`, as the converter
    does), quantised q4_0. tie_all: every centroid row the same bytes, so the choice
    of clusters is decided by the quickselect's steps alone."""
    assert NC * CS >= V
    rng = np.random.default_rng(40_000 + seed)
    ids = np.full(NC * CS, -1, np.int32)
    ids[:V] = rng.permutation(V).astype(np.int32)
    rng.shuffle(ids)                             # padding slots spread over the clusters
    tmap = ids.reshape(NC, CS)
    emb = dequant_q40(table, V, D)
    cent = np.zeros((NC, D), np.float32)
    cscale = np.zeros(NC, np.float32)
    for c in range(NC):
        m = tmap[c][tmap[c] >= 0]
        rows = emb[m]
        nrm = np.linalg.norm(rows, axis=1)
        cscale[c] = nrm.max() if m.size else 1.0
        u = (rows / np.maximum(nrm, 1e-12)[:, None]).mean(0) if m.size else np.ones(D, np.float32)
        u = u / max(np.linalg.norm(u), 1e-12)
        cent[c] = u * (cscale[c] if scaled else 1.0)
    if tie_all:
        cent[:] = cent[0]
    force = rng.choice(V, nforce, replace=False).astype(np.int32) if nforce else np.zeros(0, np.int32)
    return Flash(quant_rows(FMT_Q40, cent), NC, np.ascontiguousarray(tmap), CS, NP, cscale, scaled, force)


def _flash_argtypes(extra_sel):
    base = [u8p, C.c_int, C.c_int, f32p, C.c_float, C.c_float, u8p, C.c_int, i32p, C.c_int, C.c_int,
            f32p, C.c_int, i32p, C.c_int, f32p, f32p]
    return base + ([i32p] if extra_sel else [])


# A FlashHead over a 4032-row table: 128 balanced clusters of 32 (64 padding slots),
# 14 probed, 3 forced ids. tie_all makes every centroid the same bytes, so the probed
# set is decided by the quickselect's steps alone (the case a plain top-k would get
# wrong).
FLASH_CASE = dict(V=4032, D=1024, NC=128, CS=32, NP=14, nforce=3)


def flash_case(scaled=1, tie_all=False):
    """(table, final norm, Flash, H [3, D]) of the FlashHead test case."""
    f = FLASH_CASE
    table, fnorm = make_table(f["V"], f["D"], 7)
    F = make_flash(table, f["V"], f["D"], f["NC"], f["CS"], f["NP"], f["nforce"], seed=1,
                   scaled=scaled, tie_all=tie_all)
    L = make_layer("gemma", seed=1, E=8, D=f["D"], MI=64, K=2)
    H = make_input(L, 3, 9)
    return table, fnorm, F, H


def oracle_flash(table, V, D, fnorm, eps, cap, F, H):
    """(logits [S, V], greedy [S], chosen clusters [S, NP] sorted) of orc_flash_head."""
    L = oracle()
    L.orc_flash_head.argtypes = _flash_argtypes(True)
    H = np.ascontiguousarray(H, np.float32)
    S = H.shape[0]
    lg = np.zeros((S, V), np.float32)
    sel = np.zeros((S, F.NP), np.int32)
    force = F.force if F.nforce else np.zeros(1, np.int32)
    am = np.array([L.orc_flash_head(ptr(table), V, D, ptr(fnorm), C.c_float(eps), C.c_float(cap),
                                    ptr(F.cent), F.NC, ptr(F.tmap), F.CS, F.NP, ptr(F.cscale), F.scaled,
                                    ptr(force), F.nforce, ptr(H[s]), ptr(lg[s]), ptr(sel[s]))
                   for s in range(S)], np.int32)
    return lg, am, sel


def ref_flash(table, V, D, fnorm, eps, cap, F, H):
    """The compiled reference's flash_logits + sample, or None where it is unavailable."""
    lib = ref_lib("gemma4")
    if lib is None:
        return None
    lib.ref_g4_flash.argtypes = _flash_argtypes(False)
    H = np.ascontiguousarray(H, np.float32)
    S = H.shape[0]
    lg = np.zeros((S, V), np.float32)
    force = F.force if F.nforce else np.zeros(1, np.int32)
    am = np.array([lib.ref_g4_flash(ptr(table), V, D, ptr(fnorm), C.c_float(eps), C.c_float(cap),
                                    ptr(F.cent), F.NC, ptr(F.tmap), F.CS, F.NP, ptr(F.cscale), F.scaled,
                                    ptr(force), F.nforce, ptr(H[s]), ptr(lg[s]))
                   for s in range(S)], np.int32)
    return lg, am


@dataclass
class Stack:
    """A seeded gemma stack: per layer a MoE layer and a dense branch, plus the tied
    head (BASELINE config 5 with attention as the identity)."""
    layers: list
    denses: list
    table: np.ndarray
    fnorm: np.ndarray
    V: int
    embed_scale: float
    softcap: float = 30.0


def make_stack(n_layers, D, MI, E, K, DI, V, seed, zipf=False):
    layers = [make_layer("gemma", seed=100 * seed + l, E=E, D=D, MI=MI, K=K, zipf=zipf)
              for l in range(n_layers)]
    denses = [make_dense(D, DI, 100 * seed + l) for l in range(n_layers)]
    table, fnorm = make_table(V, D, seed)
    return Stack(layers, denses, table, fnorm, V, float(np.sqrt(np.float32(D))))


def stack_run(st, H0, n_decode, block, head, embed):
    """Prefill H0 through every layer, then n_decode greedy steps; the per-layer and
    head functions are passed in (oracle or compiled reference). Returns the tokens,
    the prefill output and the last decode step's logits."""
    H = np.array(H0, np.float32, copy=True)
    for L_, dn in zip(st.layers, st.denses):
        H = block(L_, dn, H)[0]
    Hp = H.copy()
    lg, am = head(st.table, st.V, st.layers[0].D, st.fnorm, st.layers[0].eps, st.softcap, H[-1:])
    toks = [int(am[0])]
    for _ in range(n_decode):
        H = embed(st.table, st.V, st.layers[0].D, st.embed_scale, toks[-1:])
        for L_, dn in zip(st.layers, st.denses):
            H = block(L_, dn, H)[0]
        lg, am = head(st.table, st.V, st.layers[0].D, st.fnorm, st.layers[0].eps, st.softcap, H)
        toks.append(int(am[0]))
    return np.array(toks, np.int32), Hp, lg[0]


def oracle_stack(st, H0, n_decode):
    return stack_run(st, H0, n_decode, oracle_block, oracle_head,
                     lambda t, V, D, s, tk: oracle_embed(t, D, s, tk))


def ref_stack(st, H0, n_decode):
    if ref_lib("gemma4") is None:
        return None
    return stack_run(st, H0, n_decode, ref_block, ref_head, ref_embed)


# ---------------------------------------- the golden gemma fixture's case
# (tests/golden/gemma_block_stack.npz, written by tests/golden/make_golden.py)
def _input_digest(L, x):
    import hashlib
    h = hashlib.sha256()
    for a in (L.router, L.router_scale, L.pes, L.bias, L.pre_ln, L.post_ln, L.experts, x):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---------------------------------------------- the Zipf offset, through the reference
# configs[1] adds a seeded Zipf(1.1) offset to each gemma logit after the in-order
# chain: v = fl(chain + bias[e]). The reference router has no offset
# (gemma4.c:600-601), but its chain's last product can carry one exactly: with every
# input element +-1 and eps = 0 the rmsnorm factor is exactly 1 (gemma4.c:425-431),
# so the router input of a last element x = 1 with router_scale 1 is exactly
# rs = 1/sqrtf(D), and a router weight q = fl(zipf / rs) gives the product
# fl(q * rs), which is taken as the offset. The reference's chain then ends with
# "+ offset", which is the oracle's faithful form and none of the plausible slips.
ZIPF_PIN = dict(seed=41, E=128, D=2816, MI=704, K=8, S=8, xseed=41)


def pm1_input(S, D, seed, last_one=True):
    """[S, D] of +-1 (the last element +1): the rmsnorm factor is exactly 1 at eps 0."""
    rng = np.random.default_rng(20_000 + seed)
    x = np.where(rng.random((S, D)) < 0.5, np.float32(-1), np.float32(1)).astype(np.float32)
    if last_one:
        x[:, D - 1] = 1.0
    return x


def zipf_pin_case(seed=41, E=128, D=2816, MI=704, K=8, S=8, xseed=41):
    """(Lo, Lr, x): Lo a Zipf-offset gemma layer for the oracle and the GPU (its last
    router column zero, so its chain over D elements is the chain over D - 1 plus an
    exact +0), Lr the same layer for the reference with the offset in that column
    and no offset of its own, x the +-1 input."""
    import dataclasses
    Lo = make_layer("gemma", seed=seed, E=E, D=D, MI=MI, K=K, zipf=True)
    Lo.eps = 0.0
    rs = np.float32(1.0) / np.sqrt(np.float32(D))
    q = (Lo.bias / rs).astype(np.float32)
    Lo.bias = (q * rs).astype(np.float32)
    Lo.router_scale = Lo.router_scale.copy()
    Lo.router_scale[D - 1] = 1.0
    Lr = dataclasses.replace(Lo, use_bias=0, bias=None, router=Lo.router.copy(), _keep=[])
    Lr.router[:, D - 1] = q
    Lo.router = Lo.router.copy()
    Lo.router[:, D - 1] = 0.0
    return Lo, Lr, pm1_input(S, D, xseed)


# gemma around the MoE block: (D, MI, E, K, DI, V, seed), the block's S, the stack's
# layers, prefill rows and greedy steps, and the embedding scale of the stack case
GEMMA_SHAPE = (512, 256, 16, 4, 512, 1024, 3)
GEMMA_BLOCK_S = 6
GEMMA_STACK = dict(layers=2, S=6, steps=6, embed_scale=1.0)
GEMMA_TOKS = [0, 1, 17, 511, 1023]


def gemma_block_case():
    """What the golden gemma fixture's inputs are, regenerated from seeds."""
    D, MI, E, K, DI, V, seed = GEMMA_SHAPE
    L = make_layer("gemma", seed=seed, E=E, D=D, MI=MI, K=K)
    dn = make_dense(D, DI, seed)
    H = make_input(L, GEMMA_BLOCK_S, seed)
    table, fnorm = make_table(V, D, seed)
    st = make_stack(GEMMA_STACK["layers"], D, MI, E, K, DI, V, seed)
    st.embed_scale = GEMMA_STACK["embed_scale"]
    H0 = make_input(L, GEMMA_STACK["S"], seed + 1)
    return L, dn, H, table, fnorm, st, H0


def gemma_digest(L, dn, H, table, fnorm, st, H0):
    import hashlib
    h = hashlib.sha256()
    h.update(_input_digest(L, H).encode())
    for a in (dn.mlp, dn.pre_ffn_ln, dn.post_ffn_ln1, dn.post_ffn_ln, table, fnorm, H0):
        h.update(np.ascontiguousarray(a).tobytes())
    for l_, d_ in zip(st.layers, st.denses):
        h.update(_input_digest(l_, H0).encode())
        h.update(np.ascontiguousarray(d_.mlp).tobytes())
    return h.hexdigest()


# ------------------------------------------------ zunzuncito container directories
def write_gemma_container(path, st, head_dim=64, n_heads=2, flash=None):
    """Write stack `st` as a gemma4 container directory in the layout that
    tools/convert_gemma4.py writes and gemma4.c:260-403 reads: manifest.txt (cfg
    lines, `esz`, the dense index, `expert li e off`), dense.bin (tensors back to
    back: q4_0 matrices, f32 vectors, shapes [O, I] with I = 1 for vectors) and
    experts.bin ([gate | up | down] records at 4096-aligned offsets). Attention
    tensors are small seeded placeholders: the engine's reader binds them, the GPU
    loader skips them. `flash` (a Flash) adds the FlashHead tensors and cfg keys as
    convert_gemma4.py:315-327, 400 writes them. Returns the per-(layer, expert)
    offsets."""
    os.makedirs(path, exist_ok=True)
    L0 = st.layers[0]
    D, MI, E, K, NL = L0.D, L0.MI, L0.E, L0.K, len(st.layers)
    DI = st.denses[0].DI
    rng = np.random.default_rng(4242)
    dense, off = [], 0
    blob = open(os.path.join(path, "dense.bin"), "wb")

    def add(name, arr, fmt, O, I):
        nonlocal off
        b = np.ascontiguousarray(arr).tobytes()
        blob.write(b)
        dense.append((name, off, len(b), fmt, O, I))
        off += len(b)

    def q40(O, I):
        return make_expert_q(rng, FMT_Q40, O, I)

    add("embed_tokens", st.table, 1, st.V, D)
    add("norm", st.fnorm, 0, D, 1)
    for l, (L_, dn) in enumerate(zip(st.layers, st.denses)):
        o = f"layers.{l}."
        ones = np.ones(D, np.float32)
        for nm, v in (("input_layernorm", ones), ("post_attention_layernorm", ones),
                      ("pre_feedforward_layernorm", dn.pre_ffn_ln),
                      ("post_feedforward_layernorm", dn.post_ffn_ln),
                      ("pre_feedforward_layernorm_2", L_.pre_ln),
                      ("post_feedforward_layernorm_1", dn.post_ffn_ln1),
                      ("post_feedforward_layernorm_2", L_.post_ln)):
            add(o + nm, v, 0, D, 1)
        add(o + "layer_scalar", np.array([dn.layer_scalar], np.float32), 0, 1, 1)
        hd = head_dim
        add(o + "q_proj", q40(n_heads * hd, D), 1, n_heads * hd, D)
        add(o + "k_proj", q40(hd, D), 1, hd, D)
        add(o + "v_proj", q40(hd, D), 1, hd, D)
        add(o + "o_proj", q40(D, n_heads * hd), 1, D, n_heads * hd)
        add(o + "q_norm", np.ones(hd, np.float32), 0, hd, 1)
        add(o + "k_norm", np.ones(hd, np.float32), 0, hd, 1)
        gb = tensor_bytes(FMT_Q40, DI, D)
        add(o + "mlp_gate", dn.mlp[:gb], 1, DI, D)
        add(o + "mlp_up", dn.mlp[gb:2 * gb], 1, DI, D)
        add(o + "mlp_down", dn.mlp[2 * gb:], 1, D, DI)
        add(o + "router_proj", L_.router, 0, E, D)
        add(o + "router_scale", L_.router_scale, 0, D, 1)
        add(o + "router_pes", L_.pes, 0, E, 1)
    if flash is not None:
        add("flash_centroids", flash.cent, 1, flash.NC, D)
        add("flash_token_map", flash.tmap, 5, flash.NC, flash.CS)
        add("flash_cluster_scale", flash.cscale, 0, 1, flash.NC)
        fo = flash.force if flash.nforce else np.zeros(1, np.int32)
        add("flash_force", fo.astype(np.int32), 5, 1, fo.size)
    blob.close()
    esz, gb, db = L0.esz, tensor_bytes(FMT_Q40, MI, D), tensor_bytes(FMT_Q40, D, MI)
    eoff, off = {}, 0
    with open(os.path.join(path, "experts.bin"), "wb") as f:
        for l, L_ in enumerate(st.layers):
            for e in range(E):
                pad = (-off) % 4096
                f.write(b"\0" * pad)
                off += pad
                f.write(L_.experts[e * esz:(e + 1) * esz].tobytes())
                eoff[(l, e)] = off
                off += esz
    cfg = dict(hidden=D, n_layers=NL, n_heads=n_heads, head_dim=head_dim, global_head_dim=head_dim,
               n_kv_heads=1, n_global_kv_heads=1, k_eq_v_global=False, n_experts=E, topk=K,
               moe_inter=MI, dense_inter=DI, vocab=st.V, eps=L0.eps, sliding_window=128,
               rope_theta_local=10000.0, rope_theta_global=1000000.0, rope_partial_global=1.0,
               final_logit_softcap=st.softcap, embed_scale=st.embed_scale, ctx=256,
               slots_per_layer=E)
    if flash is not None:
        cfg.update(flash_n_clusters=flash.NC, flash_cluster_size=flash.CS, flash_n_probes=flash.NP,
                   flash_scaled_centroids=flash.scaled, flash_n_force=flash.nforce)
    with open(os.path.join(path, "manifest.txt"), "w") as m:
        for k, v in cfg.items():
            m.write(f"cfg {k} {v}\n")
        m.write("cfg layer_types " + " ".join("0" for _ in range(NL)) + "\n")
        m.write(f"esz {esz} {gb} {db}\n")
        m.write(f"ndense {len(dense)}\n")
        for name, o_, ln, fmt, O, I in dense:
            m.write(f"dense {name} {o_} {ln} {fmt} {O} {I}\n")
        m.write(f"nexpert {len(eoff)}\n")
        for (l, e), o_ in eoff.items():
            m.write(f"expert {l} {e} {o_}\n")
    return eoff


def write_moe_container(path, layers, per_layer):
    """The expert part of a container directory for MoE layers `layers`: experts.bin
    ([gate | up | down] records at 4096-aligned offsets, as tools/convert_*.py write
    them) and a manifest.txt with the model cfg, the record size -- one `esz` line
    (maple.c:255-258, gemma) or, with per_layer, one `eszl li esz gate down fmt` line
    per layer with the layer's expert format (lfm25.c:328-331, convert_lfm25.py:490)
    -- and one `expert li e off` line per record. Returns the offsets."""
    os.makedirs(path, exist_ok=True)
    eoff, off = {}, 0
    with open(os.path.join(path, "experts.bin"), "wb") as f:
        for li, L_ in enumerate(layers):
            for e in range(L_.E):
                pad = (-off) % 4096
                f.write(b"\0" * pad)
                off += pad
                f.write(L_.experts[e * L_.esz:(e + 1) * L_.esz].tobytes())
                eoff[(li, e)] = off
                off += L_.esz
    L0 = layers[0]
    with open(os.path.join(path, "manifest.txt"), "w") as m:
        for k, v in dict(hidden=L0.D, n_layers=len(layers), n_experts=L0.E, topk=L0.K,
                         moe_inter=L0.MI).items():
            m.write(f"cfg {k} {v}\n")
        if per_layer:
            for li, L_ in enumerate(layers):
                g, _, d = L_.tensor_sizes()
                m.write(f"eszl {li} {L_.esz} {g} {d} {L_.fmts[0]}\n")
        else:
            g, _, d = L0.tensor_sizes()
            m.write(f"esz {L0.esz} {g} {d}\n")
        m.write("ndense 0\n")
        m.write(f"nexpert {len(eoff)}\n")
        for (li, e), o in eoff.items():
            m.write(f"expert {li} {e} {o}\n")
    return eoff
