"""Pins for the oracle's gemma pieces around the MoE block (oracle/zz_oracle.c:
orc_dense_mlp, orc_gemma_ffn_block, orc_embed_row, orc_head): the feed-forward half
of layer_fwd (gemma4.c:1003-1030), embed_row (gemma4.c:1131-1145), the tied head
(gemma4.c:1264-1275) and greedy selection (gemma4.c:2149-2152).

Each is checked against the compiled reference's fixture (tests/golden/
gemma_block_stack.npz, written by oracle/_ref through the engine's own functions),
live against oracle/_ref where it is built, and against closed forms that share no
code with it: numpy dequantisation, a float64 dot product, np.argmax's first-index
rule, and the identity "dense branch = one-expert MoE layer at weight 1".
"""
import ctypes as C
import os

import numpy as np
import pytest

import zzref as Z

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma_block_stack.npz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def case():
    g = np.load(GOLDEN)
    L, dn, H, table, fnorm, st, H0 = Z.gemma_block_case()
    assert Z.gemma_digest(L, dn, H, table, fnorm, st, H0) == str(g["digest"]), \
        "input generator drifted from the fixture"
    return g, L, dn, H, table, fnorm, st, H0


def test_block_golden_bit_exact(case):
    g, L, dn, H, *_ = case
    Hb, eidx, ewt = Z.oracle_block(L, dn, H)
    assert np.array_equal(eidx, g["block_eidx"])
    assert np.array_equal(bits(ewt), bits(g["block_ewt"]))
    assert np.array_equal(bits(Hb), bits(g["block_H"]))


def test_embed_and_head_golden_bit_exact(case):
    g, L, dn, H, table, fnorm, st, H0 = case
    D, V = L.D, Z.GEMMA_SHAPE[5]
    emb = Z.oracle_embed(table, D, np.float32(np.sqrt(np.float32(D))), Z.GEMMA_TOKS)
    assert np.array_equal(bits(emb), bits(g["embed"]))
    lg, am = Z.oracle_head(table, V, D, fnorm, L.eps, 30.0, H[:3])
    assert np.array_equal(bits(lg), bits(g["head_logits"]))
    assert np.array_equal(am, g["head_argmax"])


def test_stack_golden_bit_exact(case):
    g, *_, st, H0 = case
    toks, Hp, lg = Z.oracle_stack(st, H0, Z.GEMMA_STACK["steps"])
    assert np.array_equal(toks, g["stack_tokens"])
    assert np.array_equal(bits(Hp), bits(g["stack_prefill"]))
    assert np.array_equal(bits(lg), bits(g["stack_logits"]))
    assert len(set(toks.tolist())) > 2            # the greedy walk is not a fixed point


def test_block_vs_compiled_reference():
    """Live diff at another shape and seed (Zipf offsets are a harness extension the
    reference cannot express, so the router is the plain one here)."""
    if Z.ref_lib("gemma4") is None:
        pytest.skip("oracle/_ref not built here")
    L = Z.make_layer("gemma", seed=41, E=24, D=1024, MI=512, K=6)
    dn = Z.make_dense(1024, 768, 41)
    H = Z.make_input(L, 9, 41)
    a, b = Z.oracle_block(L, dn, H), Z.ref_block(L, dn, H)
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(bits(a[0]), bits(b[0]))


def test_dense_branch_is_one_expert_moe():
    """The dense MLP (gemma4.c:1012-1020) is the expert FFN (gemma4.c:618-654) of a
    one-expert layer routed at weight 1 (softmax of one logit is 1, pes = 1, and
    fma(1, y, 0) = y), with pre_ffn_ln / post_ffn_ln1 as the two norms."""
    D, DI = 512, 512
    dn = Z.make_dense(D, DI, 5)
    L = Z.Layer(D, DI, 1, 1, Z.GATE_GEMMA, Z.ACT_GEGLU_TANH, (Z.FMT_Q40,) * 3, eps=1e-6)
    L.router = np.zeros((1, D), np.float32)
    L.router_scale = np.ones(D, np.float32)
    L.pes = np.ones(1, np.float32)
    L.pre_ln, L.post_ln = dn.pre_ffn_ln, dn.post_ffn_ln1
    L.experts, L.esz = dn.mlp, dn.mlp.size
    x = Z.make_input(L, 7, 5)
    want = Z.oracle_moe(L, x).out
    got = Z.oracle_dense(dn, 1e-6, x)
    assert np.array_equal(bits(got), bits(want))


def dequant_q40(table, V, D):
    b = table.reshape(V, D // 32, 18)
    d = b[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    q = b[:, :, 2:]
    lo = (q & 15).astype(np.int32) - 8
    hi = (q >> 4).astype(np.int32) - 8
    return d, np.concatenate([lo, hi], axis=2)        # [V, nb], [V, nb, 32]


def test_embed_closed_form():
    V, D = 256, 512
    table, _ = Z.make_table(V, D, 9)
    d, q = dequant_q40(table, V, D)
    scale = np.float32(22.627417)
    toks = [0, 5, 255, 128]
    want = ((d[toks][:, :, None] * q[toks].astype(np.float32)).astype(np.float32) * scale).reshape(len(toks), D)
    got = Z.oracle_embed(table, D, scale, toks)
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))


def test_head_closed_form_and_first_index_argmax():
    """Logits = softcap(sum_b d_w d_x <q-8, xq>) to float rounding (float64 here);
    the greedy token is the first index of the maximum, also when values tie."""
    V, D = 512, 512
    table, fnorm = Z.make_table(V, D, 11)
    h = Z.make_input(Z.make_layer("gemma", seed=1, E=8, D=D, MI=64, K=2), 1, 11)
    L = Z.oracle()
    L.orc_rmsnorm.argtypes = [Z.f32p, Z.f32p, Z.f32p, C.c_int, C.c_float]
    xn = np.zeros(D, np.float32)
    L.orc_rmsnorm(Z.ptr(xn), Z.ptr(h[0]), Z.ptr(fnorm), D, C.c_float(1e-6))
    xq = np.zeros(D, np.int8)
    xs = np.zeros(D // 32, np.float32)
    L.orc_quant_act(Z.ptr(xn), Z.ptr(xq), Z.ptr(xs), D)
    d, q = dequant_q40(table, V, D)
    dots = (q * xq.reshape(D // 32, 32)[None].astype(np.int32)).sum(axis=2)
    raw = (d.astype(np.float64) * xs[None].astype(np.float64) * dots).sum(axis=1)
    for cap in (0.0, 30.0):
        lg, am = Z.oracle_head(table, V, D, fnorm, 1e-6, cap, h)
        want = np.tanh(raw / cap) * cap if cap > 0 else raw
        assert np.allclose(lg[0], want, rtol=1e-5, atol=1e-5)
        assert am[0] == int(np.argmax(lg[0]))
    # duplicate the winning row at a later index: the first one still wins
    t2 = table.reshape(V, -1).copy()
    t2[V - 1] = t2[am[0]]
    lg2, am2 = Z.oracle_head(t2.reshape(-1), V, D, fnorm, 1e-6, 30.0, h)
    assert lg2[0, V - 1] == lg2[0, am[0]] and am2[0] == am[0]


def test_block_tolerance_is_discriminating():
    """A slip in the combine (post_ffn_ln1 for post_ffn_ln, or a dropped layer
    scalar) moves the block output far beyond the GPU tier's 1e-3."""
    L = Z.make_layer("gemma", seed=3, E=16, D=512, MI=256, K=4)
    dn = Z.make_dense(512, 512, 3)
    H = Z.make_input(L, 6, 3)
    good = Z.oracle_block(L, dn, H)[0]
    bad = Z.Dense(dn.D, dn.DI, dn.mlp, dn.pre_ffn_ln, dn.post_ffn_ln1, dn.post_ffn_ln1, dn.layer_scalar)
    assert Z.rel_l2(Z.oracle_block(L, bad, H)[0], good) > 1e-2
    bad2 = Z.Dense(dn.D, dn.DI, dn.mlp, dn.pre_ffn_ln, dn.post_ffn_ln1, dn.post_ffn_ln, 1.0)
    assert Z.rel_l2(Z.oracle_block(L, bad2, H)[0], good) > 1e-2


def test_container_writer_read_by_the_engine(tmp_path):
    """The test-side container writer (zzref.write_gemma_container) produces what the
    engine's own reader, manifest() (gemma4.c:260-403), parses back: record size,
    every expert offset, the dense tensors by name, and the expert bytes at the
    engine's offsets. The GPU loader is then tested against the same directories."""
    lib = Z.ref_lib("gemma4")
    if lib is None:
        pytest.skip("oracle/_ref not built here")
    *_, st, H0 = Z.gemma_block_case()
    eoff = Z.write_gemma_container(str(tmp_path), st)
    L0, NL = st.layers[0], len(st.layers)
    D, E = L0.D, L0.E
    lib.ref_g4_manifest_probe.argtypes = [C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                          Z.f32p, Z.f32p, Z.f32p, Z.u8p, C.c_int, C.c_int, Z.u8p]
    esz3 = np.zeros(3, np.int64)
    eo = np.zeros(NL * E, np.int64)
    r0 = np.zeros((E, D), np.float32)
    sc = np.zeros(NL, np.float32)
    fn = np.zeros(D, np.float32)
    row0 = np.zeros(D // 32 * 18, np.uint8)
    rec = np.zeros(L0.esz, np.uint8)
    li, e = NL - 1, E - 3
    nl = lib.ref_g4_manifest_probe(str(tmp_path).encode(), esz3.ctypes.data_as(C.POINTER(C.c_int64)),
                                   eo.ctypes.data_as(C.POINTER(C.c_int64)), Z.ptr(r0), Z.ptr(sc),
                                   Z.ptr(fn), Z.ptr(row0), li, e, Z.ptr(rec))
    assert nl == NL
    assert esz3.tolist() == [L0.esz, Z.tensor_bytes(1, L0.MI, D), Z.tensor_bytes(1, D, L0.MI)]
    assert eo.tolist() == [eoff[(l, x)] for l in range(NL) for x in range(E)]
    assert all(o % 4096 == 0 for o in eo)
    assert np.array_equal(r0, st.layers[0].router)
    assert np.array_equal(sc, np.array([d.layer_scalar for d in st.denses], np.float32))
    assert np.array_equal(fn, st.fnorm)
    assert np.array_equal(row0, st.table[:row0.size])
    assert np.array_equal(rec, st.layers[li].experts[e * L0.esz:(e + 1) * L0.esz])


# ------------------------------------------------------------------- FlashHead
FLASH = Z.FLASH_CASE
FLASH_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma_flash_head.npz")
flash_case = Z.flash_case


def probed_ids(F, sel, V):
    ids = set(int(i) for c in sel for i in F.tmap[c] if 0 <= i < V)
    return ids | set(int(i) for i in F.force)


@pytest.mark.parametrize("scaled,tie_all", [(1, False), (0, False), (1, True)])
def test_flash_head_vs_compiled_reference(scaled, tie_all):
    """orc_flash_head against the engine's own flash_logits + sample, bit for bit."""
    table, fnorm, F, H = flash_case(scaled, tie_all)
    V, D = FLASH["V"], FLASH["D"]
    ref = Z.ref_flash(table, V, D, fnorm, 1e-6, 30.0, F, H)
    if ref is None:
        pytest.skip("oracle/_ref not built")
    lg, am, sel = Z.oracle_flash(table, V, D, fnorm, 1e-6, 30.0, F, H)
    assert np.array_equal(bits(lg), bits(ref[0]))
    assert np.array_equal(am, ref[1])
    for s in range(H.shape[0]):
        fin = set(np.flatnonzero(np.isfinite(lg[s])).tolist())
        assert fin == probed_ids(F, sel[s], V)


def test_flash_head_probing_every_cluster_is_the_full_head():
    """With every cluster probed (NP = NC) and no forced ids, the flash logits are the
    full head's: same dots, same softcap, every id a member of some cluster."""
    table, fnorm, F, H = flash_case()
    V, D = FLASH["V"], FLASH["D"]
    F.NP, F.force = F.NC, np.zeros(0, np.int32)
    lg, am, sel = Z.oracle_flash(table, V, D, fnorm, 1e-6, 30.0, F, H)
    full, fam = Z.oracle_head(table, V, D, fnorm, 1e-6, 30.0, H)
    assert np.array_equal(bits(lg), bits(full)) and np.array_equal(am, fam)
    assert np.array_equal(sel[0], np.arange(F.NC))


def test_flash_head_picks_the_best_clusters():
    """Without ties the probed set is the NP clusters of largest score, whatever the
    quickselect's order: checked against a float64 score's ranking, away from ties."""
    table, fnorm, F, H = flash_case()
    V, D = FLASH["V"], FLASH["D"]
    _, _, sel = Z.oracle_flash(table, V, D, fnorm, 1e-6, 30.0, F, H)
    cent = Z.dequant_q40(F.cent, F.NC, D).astype(np.float64)
    for s in range(H.shape[0]):
        h = H[s].astype(np.float64)
        xn = h / np.sqrt(np.mean(h * h) + 1e-6) * fnorm
        score = cent @ xn
        order = np.argsort(-score)
        gap = score[order[F.NP - 1]] - score[order[F.NP]]
        if gap > 1e-3 * np.abs(score).max():
            assert np.array_equal(np.sort(order[:F.NP]), sel[s])


def test_flash_head_golden():
    """The fixture the compiled reference wrote (tests/golden/make_golden.py)."""
    g = np.load(FLASH_GOLDEN)
    for key, (scaled, tie_all) in (("plain", (1, False)), ("ties", (1, True))):
        table, fnorm, F, H = flash_case(scaled, tie_all)
        lg, am, sel = Z.oracle_flash(table, FLASH["V"], FLASH["D"], fnorm, 1e-6, 30.0, F, H)
        assert np.array_equal(am, g[f"{key}_argmax"])
        assert np.array_equal(sel, g[f"{key}_sel"])
        fin = np.isfinite(lg)
        assert np.array_equal(fin, g[f"{key}_finite"])
        assert np.array_equal(bits(lg[fin]), bits(g[f"{key}_logits"]))
