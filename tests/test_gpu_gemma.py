"""GPU parity for gemma's pieces around the MoE block (include/zz_gemma.h and the
ZZ_GATE_DENSE layer kind), against the oracle and the compiled reference's fixture
(tests/golden/gemma_block_stack.npz):

  bit-exact  the dense branch's int8 activations, the MoE routing inside a block,
             embed_row;
  fp32       dense-branch and block outputs within 1e-3 relative L2; logits within
             1e-3 of the logit scale; the greedy token equal wherever the oracle's
             top-two margin exceeds that tolerance.
A whole stack (prefill then greedy decode on the device, token ids never leaving
it) is checked step by step against the oracle fed the GPU's own tokens.
"""
import sys

import numpy as np
import pytest

import zzref as Z
import zunzuncito_amd as zz

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-3
LOGIT_TOL = 1e-3          # absolute, logits are O(1..30)


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def dev():
    return zz.init()


def gpu_moe(L):
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, L.bias, L.pre_ln, L.post_ln, use_bias=L.use_bias, eps=L.eps)
    m.upload_all(L.experts)
    return m


def gpu_dense(dn, eps=1e-6):
    m = zz.MoeLayer(dn.D, dn.DI, 1, 1, zz.ZZ_GATE_DENSE, zz.ZZ_ACT_GEGLU_TANH, (1, 1, 1), None,
                    pre_ln=dn.pre_ffn_ln, post_ln=dn.post_ffn_ln1, eps=eps)
    m.upload(0, dn.mlp)
    return m


def gpu_block(L, dn):
    m, d = gpu_moe(L), gpu_dense(dn)
    return zz.FfnBlock(m, d, dn.post_ffn_ln, dn.layer_scalar), m, d


def close_all(*objs):
    for o in objs:
        o.close()


@pytest.mark.parametrize("D,DI,S", [(512, 512, 1), (512, 512, 3), (512, 512, 40),
                                    (2816, 2112, 1), (2816, 2112, 64)])
def test_dense_branch(dev, D, DI, S):
    """ZZ_GATE_DENSE on the decode (S <= 4) and matrix-core paths: every row to
    expert 0 at weight 1, int8 activations bit-exact, outputs within 1e-3."""
    say(f"dense D={D} DI={DI} S={S}")
    dn = Z.make_dense(D, DI, 8)
    L = Z.make_layer("gemma", seed=1, E=8, D=D, MI=64, K=2)
    x = Z.make_input(L, S, 8)
    m = gpu_dense(dn)
    try:
        out, eidx, ewt = m.forward(x)
        assert np.all(eidx == 0) and np.all(ewt == 1.0)
        want = Z.oracle_dense(dn, 1e-6, x)
        err = Z.rel_l2(out, want)
        say(f"  rel L2 {err:.2e}")
        assert err < OUT_TOL, err
        # the int8 expert input: q8_0 of rmsnorm(x, pre_ffn_ln)
        d = m.debug(S)
        O = Z.oracle()
        for s in range(S):
            xn = np.zeros(D, np.float32)
            O.orc_rmsnorm.argtypes = [Z.f32p, Z.f32p, Z.f32p, Z.C.c_int, Z.C.c_float]
            O.orc_rmsnorm(Z.ptr(xn), Z.ptr(x[s]), Z.ptr(dn.pre_ffn_ln), D, Z.C.c_float(1e-6))
            xq = np.zeros(D, np.int8)
            xs = np.zeros(D // 32, np.float32)
            O.orc_quant_act(Z.ptr(xn), Z.ptr(xq), Z.ptr(xs), D)
            assert np.array_equal(d["xq"][s], xq)
            assert np.array_equal(d["xs"][s].view(np.uint32), xs.view(np.uint32))
    finally:
        m.close()


def test_dense_items_spread_over_xcds(dev):
    """The dense branch at S=512 is one expert of 8 work items: no placement of
    whole experts balances 8 XCDs, so its items run one per XCD in union order."""
    say("dense gemma shape S=512 items")
    dn = Z.make_dense(2816, 2112, 8)
    L = Z.make_layer("gemma", seed=1, E=8, D=2816, MI=64, K=2)
    x = Z.make_input(L, 512, 9)
    m = gpu_dense(dn)
    try:
        out, _, _ = m.forward(x)
        err = Z.rel_l2(out, Z.oracle_dense(dn, 1e-6, x))
        say(f"  rel L2 {err:.2e}")
        assert err < OUT_TOL, err
        d = m.debug(512)
        xcds = Z.check_items(d)
        used = [slot % 8 for slot, it in enumerate(d["items"]) if it[3] > 0]
        assert len(used) == 8 and sorted(used) == list(range(8)), used
        assert xcds[0] == set(range(8))
    finally:
        m.close()


def test_block_golden(dev):
    g = np.load(Z.os.path.join(Z.ROOT, "tests", "golden", "gemma_block_stack.npz"))
    L, dn, H, table, fnorm, st, H0 = Z.gemma_block_case()
    assert Z.gemma_digest(L, dn, H, table, fnorm, st, H0) == str(g["digest"])
    B, m, d = gpu_block(L, dn)
    try:
        Hb, eidx, ewt = B.forward(H)
        assert np.array_equal(eidx, g["block_eidx"])
        np.testing.assert_allclose(ewt, g["block_ewt"], rtol=1e-4, atol=1e-6)
        err = Z.rel_l2(Hb, g["block_H"])
        say(f"block vs reference fixture: rel L2 {err:.2e}")
        assert err < OUT_TOL
    finally:
        close_all(B, m, d)


@pytest.mark.parametrize("S", [1, 4, 64])
def test_block_gemma_shape(dev, S, layer_cache):
    """The Gemma-4 layer shape (d=2816, 128 experts, top-8, MI=704, dense 2112) with
    Zipf-skewed routing, on the decode and batched paths."""
    L = layer_cache("gemma", seed=2, zipf=True)
    dn = Z.make_dense(2816, 2112, 12)
    H = Z.make_input(L, S, 12)
    B, m, d = gpu_block(L, dn)
    try:
        Hb, eidx, ewt = B.forward(H)
        want = Z.oracle_block(L, dn, H)
        assert np.array_equal(eidx, want[1])
        err = Z.rel_l2(Hb, want[0])
        say(f"block S={S}: rel L2 {err:.2e}")
        assert err < OUT_TOL
    finally:
        close_all(B, m, d)


def test_block_dev_path_matches_host(dev):
    import torch
    L, dn, H, *_ = Z.gemma_block_case()
    B, m, d = gpu_block(L, dn)
    try:
        a, ea, _ = B.forward(H)
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            dH = torch.from_numpy(H).cuda()
            de = torch.zeros(H.shape[0] * L.K, dtype=torch.int32, device="cuda")
            B.forward_dev(dH.data_ptr(), H.shape[0], de.data_ptr(), 0, st.cuda_stream)
        st.synchronize()
        assert np.array_equal(dH.cpu().numpy().view(np.uint32), a.view(np.uint32))
        assert np.array_equal(de.cpu().numpy(), ea)
    finally:
        close_all(B, m, d)


def test_head_embed_and_logits(dev):
    g = np.load(Z.os.path.join(Z.ROOT, "tests", "golden", "gemma_block_stack.npz"))
    L, dn, H, table, fnorm, *_ = Z.gemma_block_case()
    D, V = L.D, Z.GEMMA_SHAPE[5]
    hd = zz.Head(table, V, D, fnorm, L.eps, float(np.sqrt(np.float32(D))), 30.0)
    try:
        emb = hd.embed(np.array(Z.GEMMA_TOKS, np.int32))
        assert np.array_equal(emb.view(np.uint32), g["embed"].view(np.uint32))
        lg, am = hd.logits(H[:3])
        err = float(np.abs(lg - g["head_logits"]).max())
        say(f"head logits max abs err {err:.2e}")
        assert err < LOGIT_TOL
        for s in range(3):
            top2 = np.sort(g["head_logits"][s])[-2:]
            if top2[1] - top2[0] > LOGIT_TOL:
                assert am[s] == g["head_argmax"][s]
    finally:
        hd.close()


def test_head_gemma_vocab_slice(dev):
    """D=2816 with a 16384-row table, 4 rows at once."""
    table, fnorm = Z.make_table(16384, 2816, 4)
    L = Z.make_layer("gemma", seed=1, E=8, D=2816, MI=64, K=2)
    H = Z.make_input(L, 4, 4)
    hd = zz.Head(table, 16384, 2816, fnorm, 1e-6, 53.06, 30.0)
    try:
        lg, am = hd.logits(H)
        want, wam = Z.oracle_head(table, 16384, 2816, fnorm, 1e-6, 30.0, H)
        err = float(np.abs(lg - want).max())
        say(f"head V=16384 max abs err {err:.2e}")
        assert err < LOGIT_TOL
        for s in range(4):
            top2 = np.sort(want[s])[-2:]
            if top2[1] - top2[0] > LOGIT_TOL:
                assert am[s] == wam[s]
    finally:
        hd.close()


def test_stack_prefill_and_greedy_decode_on_device(dev):
    """Two layers of the fixture's stack: prefill 6 rows, then 6 greedy steps with
    the token ids kept on the device (embed -> blocks -> head -> argmax -> embed).
    Each step is compared with the oracle given the GPU's own previous token, so one
    near-tie cannot cascade; the reference's fixture fixes the prefill."""
    import torch
    g = np.load(Z.os.path.join(Z.ROOT, "tests", "golden", "gemma_block_stack.npz"))
    *_, st, H0 = Z.gemma_block_case()
    D, V = st.layers[0].D, st.V
    blocks, objs = [], []
    for L_, dn in zip(st.layers, st.denses):
        B, m, d = gpu_block(L_, dn)
        blocks.append(B)
        objs += [B, m, d]
    hd = zz.Head(st.table, V, D, st.fnorm, st.layers[0].eps, st.embed_scale, st.softcap)
    objs.append(hd)
    try:
        s = torch.cuda.current_stream().cuda_stream
        dH = torch.from_numpy(H0).cuda()
        for B in blocks:
            B.forward_dev(dH.data_ptr(), H0.shape[0], stream=s)
        Hp = dH.cpu().numpy()
        err = Z.rel_l2(Hp, g["stack_prefill"])
        say(f"stack prefill vs reference fixture: rel L2 {err:.2e}")
        assert err < 2 * OUT_TOL
        dlg = torch.zeros((1, V), dtype=torch.float32, device="cuda")
        dtok = torch.zeros(1, dtype=torch.int32, device="cuda")
        hd.logits_dev(dH[-1:].data_ptr(), 1, dlg.data_ptr(), dtok.data_ptr(), s)
        h1 = torch.zeros((1, D), dtype=torch.float32, device="cuda")
        toks = [int(dtok.item())]
        for step in range(Z.GEMMA_STACK["steps"]):
            hd.embed_dev(dtok.data_ptr(), 1, h1.data_ptr(), s)
            for B in blocks:
                B.forward_dev(h1.data_ptr(), 1, stream=s)
            hd.logits_dev(h1.data_ptr(), 1, dlg.data_ptr(), dtok.data_ptr(), s)
            # the oracle's step from the same token
            He = Z.oracle_embed(st.table, D, st.embed_scale, toks[-1:])
            for L_, dn in zip(st.layers, st.denses):
                He = Z.oracle_block(L_, dn, He)[0]
            wl, wam = Z.oracle_head(st.table, V, D, st.fnorm, st.layers[0].eps, st.softcap, He)
            got_h, got_l, tok = h1.cpu().numpy(), dlg.cpu().numpy(), int(dtok.item())
            assert Z.rel_l2(got_h, He) < 2 * OUT_TOL
            assert float(np.abs(got_l - wl).max()) < LOGIT_TOL
            top2 = np.sort(wl[0])[-2:]
            if top2[1] - top2[0] > LOGIT_TOL:
                assert tok == wam[0], (step, tok, wam[0])
            toks.append(tok)
        say("stack tokens", toks, "reference fixture", g["stack_tokens"].tolist())
    finally:
        close_all(*objs)


@pytest.mark.parametrize("n_blocks", [2, 3])
def test_stack_runner_graph_equals_eager(dev, n_blocks):
    """zz_stack_*: prefill equals the blocks run one by one; greedy decode replayed
    from a captured HIP graph equals eager launches bit for bit, on every step of
    three calls with eager work and host synchronisations between the replays. The
    residual stream alternates between two buffers as each block's combine is
    deferred into the next block: with 3 blocks the last combine writes the caller's
    buffer after it served as a router input, with 2 it ends in the second buffer."""
    import torch
    *_, st, H0 = Z.gemma_block_case()
    if n_blocks != len(st.layers):
        D_, MI_, E_, K_, DI_, V_, seed_ = Z.GEMMA_SHAPE
        st = Z.make_stack(n_blocks, D_, MI_, E_, K_, DI_, V_, seed_)
        st.embed_scale = Z.GEMMA_STACK["embed_scale"]
    D, V = st.layers[0].D, st.V
    blocks, objs = [], []
    for L_, dn in zip(st.layers, st.denses):
        B, m, d = gpu_block(L_, dn)
        blocks.append(B)
        objs += [B, m, d]
    hd = zz.Head(st.table, V, D, st.fnorm, st.layers[0].eps, st.embed_scale, st.softcap)
    stack = zz.Stack(blocks, hd)
    objs += [stack, hd]
    try:
        s = torch.cuda.current_stream().cuda_stream
        dH = torch.from_numpy(H0).cuda()
        tok0 = torch.zeros(1, dtype=torch.int32, device="cuda")
        stack.prefill_dev(dH.data_ptr(), H0.shape[0], tok0.data_ptr(), s)
        ref = torch.from_numpy(H0).cuda()
        for B in blocks:
            B.forward_dev(ref.data_ptr(), H0.shape[0], stream=s)
        torch.cuda.synchronize()
        assert torch.equal(dH.view(torch.int32), ref.view(torch.int32))
        n = 8
        runs = []
        for graph in (False, True, True, False, True):
            toks = torch.zeros(n + 1, dtype=torch.int32, device="cuda")
            toks[0] = tok0[0]
            lg = torch.zeros(V, dtype=torch.float32, device="cuda")
            stack.decode_dev(toks.data_ptr(), n, lg.data_ptr(), graph=graph, stream=s)
            torch.cuda.synchronize()
            runs.append((graph, toks.cpu().numpy(), lg.cpu().numpy()))
            junk = torch.randn(1024, device="cuda") * 2          # eager work between replays
            assert float(junk.abs().sum()) > 0
        say("stack decode tokens", runs[0][1].tolist())
        for graph, t, l in runs[1:]:
            assert np.array_equal(t, runs[0][1]), (graph, t, runs[0][1])
            assert np.array_equal(l.view(np.uint32), runs[0][2].view(np.uint32))
        # the stack defers each block's combine into the next block's router; the
        # blocks run one by one combine in their own kernel: equal bit for bit
        h1 = torch.zeros((1, D), dtype=torch.float32, device="cuda")
        dl = torch.zeros((1, V), dtype=torch.float32, device="cuda")
        dtok = tok0.clone()
        man = [int(tok0.item())]
        for _ in range(n):
            hd.embed_dev(dtok.data_ptr(), 1, h1.data_ptr(), s)
            for B in blocks:
                B.forward_dev(h1.data_ptr(), 1, stream=s)
            hd.logits_dev(h1.data_ptr(), 1, dl.data_ptr(), dtok.data_ptr(), s)
            man.append(int(dtok.item()))
        assert man == runs[0][1].tolist(), (man, runs[0][1])
        assert np.array_equal(dl.cpu().numpy()[0].view(np.uint32), runs[0][2].view(np.uint32))
        # 3 rows through the stack (the deferred path holds up to 4) and one by one
        a3 = torch.from_numpy(H0[:3]).cuda()
        b3 = a3.clone()
        t3 = torch.zeros(1, dtype=torch.int32, device="cuda")
        stack.prefill_dev(a3.data_ptr(), 3, t3.data_ptr(), s)
        for B in blocks:
            B.forward_dev(b3.data_ptr(), 3, stream=s)
        torch.cuda.synchronize()
        assert torch.equal(a3.view(torch.int32), b3.view(torch.int32))
        # prefill's greedy token is the head of the last prefill row
        wl, wam = Z.oracle_head(st.table, V, D, st.fnorm, st.layers[0].eps, st.softcap,
                                dH[-1:].cpu().numpy())
        top2 = np.sort(wl[0])[-2:]
        if top2[1] - top2[0] > LOGIT_TOL:
            assert int(tok0.item()) == wam[0]
    finally:
        close_all(*objs)


def test_stack_graph_recaptured_after_longer_prefill(dev):
    """A captured decode step holds raw pointers to the layers' workspaces and the
    blocks' rows. A longer prefill reallocates both, so the next graph decode must
    capture again: prefill 2 rows, graph decode, prefill 8 rows, graph decode, and
    the second graph decode must equal an eager decode from the same token bit for
    bit (tokens and last logits)."""
    import torch
    *_, st, H0 = Z.gemma_block_case()
    D, V = st.layers[0].D, st.V
    blocks, objs = [], []
    for L_, dn in zip(st.layers, st.denses):
        B, m, d = gpu_block(L_, dn)
        blocks.append(B)
        objs += [B, m, d]
    hd = zz.Head(st.table, V, D, st.fnorm, st.layers[0].eps, st.embed_scale, st.softcap)
    stack = zz.Stack(blocks, hd)
    objs += [stack, hd]
    n = 4
    try:
        s = torch.cuda.current_stream().cuda_stream

        def decode(tok, graph):
            toks = torch.zeros(n + 1, dtype=torch.int32, device="cuda")
            toks[0] = tok
            lg = torch.zeros(V, dtype=torch.float32, device="cuda")
            stack.decode_dev(toks.data_ptr(), n, lg.data_ptr(), graph=graph, stream=s)
            torch.cuda.synchronize()
            return toks.cpu().numpy(), lg.cpu().numpy()

        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        dH = torch.from_numpy(np.ascontiguousarray(H0[:2])).cuda()
        stack.prefill_dev(dH.data_ptr(), 2, tok.data_ptr(), s)
        t_short, _ = decode(int(tok.item()), True)
        H8 = np.random.default_rng(8).standard_normal((8, D)).astype(np.float32)
        dH8 = torch.from_numpy(H8).cuda()
        stack.prefill_dev(dH8.data_ptr(), 8, tok.data_ptr(), s)
        t8 = int(tok.item())
        tg, lgg = decode(t8, True)
        te, lge = decode(t8, False)
        say("tokens after the short prefill", t_short.tolist(), "after the long one", tg.tolist())
        assert np.array_equal(tg, te), (tg, te)
        assert np.array_equal(lgg.view(np.uint32), lge.view(np.uint32))
        tg2, lgg2 = decode(t8, True)                  # the recaptured graph, replayed
        assert np.array_equal(tg2, te) and np.array_equal(lgg2.view(np.uint32), lge.view(np.uint32))
    finally:
        close_all(*objs)


def test_container_load(dev, tmp_path):
    """zz_gemma_stack_load / zz_moe_load_experts on a container directory written in
    the converter's layout: the loaded stack decodes exactly as the stack built from
    the same weights in memory, and its prefill matches the reference fixture."""
    import torch
    g = np.load(Z.os.path.join(Z.ROOT, "tests", "golden", "gemma_block_stack.npz"))
    *_, st, H0 = Z.gemma_block_case()
    Z.write_gemma_container(str(tmp_path), st)
    loaded = zz.Stack.load(str(tmp_path))
    objs = [loaded]
    try:
        assert (loaded.n_layers, loaded.D, loaded.V) == (len(st.layers), st.layers[0].D, st.V)
        s = torch.cuda.current_stream().cuda_stream
        dH = torch.from_numpy(H0).cuda()
        tok = torch.zeros(Z.GEMMA_STACK["steps"] + 1, dtype=torch.int32, device="cuda")
        loaded.prefill_dev(dH.data_ptr(), H0.shape[0], tok.data_ptr(), s)
        loaded.decode_dev(tok.data_ptr(), Z.GEMMA_STACK["steps"], graph=True, stream=s)
        torch.cuda.synchronize()
        err = Z.rel_l2(dH.cpu().numpy(), g["stack_prefill"])
        say(f"loaded stack prefill vs reference fixture: rel L2 {err:.2e}, tokens {tok.cpu().tolist()}")
        assert err < 2 * OUT_TOL
        assert np.array_equal(tok.cpu().numpy(), g["stack_tokens"])
        # one layer's experts through zz_moe_load_experts into a fresh layer
        L1 = st.layers[1]
        m = zz.MoeLayer(L1.D, L1.MI, L1.E, L1.K, L1.gating, L1.act, L1.fmts, L1.router,
                        L1.router_scale, L1.pes, None, L1.pre_ln, L1.post_ln, eps=L1.eps)
        objs.append(m)
        m.load_experts(str(tmp_path), 1)
        x = Z.make_input(L1, 5, 77)
        out, eidx, _ = m.forward(x)
        want = Z.oracle_moe(L1, x)
        assert np.array_equal(eidx, want.eidx) and Z.rel_l2(out, want.out) < OUT_TOL
        # a record size that is not the layer's declines with the reason
        bad = zz.MoeLayer(L1.D, L1.MI * 2, L1.E, L1.K, L1.gating, L1.act, L1.fmts, L1.router,
                          L1.router_scale, L1.pes, None, L1.pre_ln, L1.post_ln, eps=L1.eps)
        objs.append(bad)
        with pytest.raises(RuntimeError, match="record"):
            bad.load_experts(str(tmp_path), 1)
    finally:
        close_all(*objs)


@pytest.mark.parametrize("S", [1, 2, 4])
def test_block_fused_decode_matches_two_stream_path(dev, S, layer_cache):
    """Decode rows run the dense branch fused into the routed layer's four launches;
    ZZ_BLOCK_FUSE=0 keeps it on its own stream. Both agree with the oracle (routing
    exact, 1e-3) and with each other to float rounding, except where the two paths'
    different summation orders put a hidden element on opposite sides of a q8_0
    rounding boundary: the int8 hidden codes of both layers then differ by 1 in
    isolated elements, each of which moves the block's output by ~1e-4."""
    import os
    L = layer_cache("gemma", seed=2, zipf=True)
    dn = Z.make_dense(2816, 2112, 13)
    H = Z.make_input(L, S, 13 + S)
    want = Z.oracle_block(L, dn, H)
    outs, hqs = [], []
    for fuse in ("1", "0"):
        os.environ["ZZ_BLOCK_FUSE"] = fuse
        try:
            B, m, d = gpu_block(L, dn)
        finally:
            os.environ.pop("ZZ_BLOCK_FUSE")
        try:
            Hb, eidx, ewt = B.forward(H)
            Hb2, eidx2, _ = B.forward(H)           # repeatable
            assert np.array_equal(Hb.view(np.uint32), Hb2.view(np.uint32))
            assert np.array_equal(eidx, want[1])
            err = Z.rel_l2(Hb, want[0])
            say(f"block S={S} fuse={fuse}: rel L2 {err:.2e}")
            assert err < OUT_TOL
            outs.append(Hb)
            hqs.append(np.concatenate([m.debug(S)["hq"].ravel(), d.debug(S)["hq"].ravel()]).astype(np.int32))
        finally:
            close_all(B, m, d)
    flips = np.abs(hqs[0] - hqs[1])
    nf = int((flips > 0).sum())
    d01 = Z.rel_l2(outs[0], outs[1])
    say(f"  fused vs two-stream: {nf} hidden flips of {flips.size}, rel L2 {d01:.2e}")
    assert flips.max() <= 1 and nf <= max(2, flips.size // 2000)
    assert d01 < 1e-5 + 2e-4 * nf


# ------------------------------------------------------------------- FlashHead
@pytest.mark.parametrize("scaled,tie_all,cap", [(1, False, 30.0), (0, False, 30.0), (1, True, 30.0),
                                                (1, False, 0.0)])
def test_flash_head_vs_oracle(dev, scaled, tie_all, cap):
    """zz_head_flash + zz_head_use_flash against orc_flash_head (pinned to the
    compiled reference's flash_logits): the same probed ids on every row (-inf
    elsewhere), their logits bit for bit without a softcap and within the tanhf
    ulp with one, the same greedy token away from near-ties. With every centroid the
    same, the probed set comes from the quickselect replay, once per row."""
    table, fnorm, F, H = Z.flash_case(scaled, tie_all)
    V, D = Z.FLASH_CASE["V"], Z.FLASH_CASE["D"]
    hd = zz.Head(table, V, D, fnorm, 1e-6, 1.0, cap)
    try:
        hd.flash(F.cent, F.NC, F.tmap, F.CS, F.NP, F.cscale, F.scaled, F.force)
        r0 = zz.flash_replays()
        hd.use_flash(True)
        lg, am = hd.logits(H)
        replays = zz.flash_replays() - r0
        want, wam, sel = Z.oracle_flash(table, V, D, fnorm, 1e-6, cap, F, H)
        fin = np.isfinite(want)
        assert np.array_equal(np.isfinite(lg), fin)
        assert np.all(lg[~fin] == -np.inf)
        if cap == 0.0:
            assert np.array_equal(lg[fin].view(np.uint32), want[fin].view(np.uint32))
        else:
            assert float(np.abs(lg[fin] - want[fin]).max()) < LOGIT_TOL
        for s in range(H.shape[0]):
            top2 = np.sort(want[s][fin[s]])[-2:]
            if top2[1] - top2[0] > LOGIT_TOL:
                assert am[s] == wam[s], (s, am[s], wam[s])
        assert replays == (H.shape[0] if tie_all else 0), replays
        hd.use_flash(False)                      # back to the full head
        full, fam = hd.logits(H)
        wf, wfam = Z.oracle_head(table, V, D, fnorm, 1e-6, cap, H)
        assert float(np.abs(full - wf).max()) < LOGIT_TOL
    finally:
        hd.close()


def test_flash_head_declines_bad_shapes(dev):
    table, fnorm, F, H = Z.flash_case()
    V, D = Z.FLASH_CASE["V"], Z.FLASH_CASE["D"]
    hd = zz.Head(table, V, D, fnorm, 1e-6, 1.0, 30.0)
    try:
        with pytest.raises(RuntimeError, match="no FlashHead"):
            hd.use_flash(True)
        with pytest.raises(RuntimeError, match="n_probes"):
            hd.flash(F.cent, F.NC, F.tmap, F.CS, F.NC + 1, F.cscale, F.scaled, F.force)
    finally:
        hd.close()


def test_stack_decode_with_flash_head(dev, tmp_path):
    """Greedy decode through the stack with the FlashHead on: eager and graph replays
    agree bit for bit, a container carrying the FlashHead (convert_gemma4.py's
    tensors, zz_gemma_stack_load) decodes the same tokens, and each step's token is
    the oracle's flash head of the oracle's hidden from the GPU's previous token."""
    import torch
    *_, st, H0 = Z.gemma_block_case()
    D, V = st.layers[0].D, st.V
    F = Z.make_flash(st.table, V, D, 32, 32, 4, 2, seed=5)
    blocks, objs = [], []
    for L_, dn in zip(st.layers, st.denses):
        B, m, d = gpu_block(L_, dn)
        blocks.append(B)
        objs += [B, m, d]
    hd = zz.Head(st.table, V, D, st.fnorm, st.layers[0].eps, st.embed_scale, st.softcap)
    hd.flash(F.cent, F.NC, F.tmap, F.CS, F.NP, F.cscale, F.scaled, F.force)
    stack = zz.Stack(blocks, hd)
    objs += [stack, hd]
    Z.write_gemma_container(str(tmp_path), st, flash=F)
    loaded = zz.Stack.load(str(tmp_path))
    objs.append(loaded)
    try:
        s = torch.cuda.current_stream().cuda_stream
        n = 6
        runs = []
        for stk, graph in ((stack, False), (stack, True), (loaded, True), (loaded, False)):
            stk.use_flash(True)
            dH = torch.from_numpy(H0).cuda()
            toks = torch.zeros(n + 1, dtype=torch.int32, device="cuda")
            stk.prefill_dev(dH.data_ptr(), H0.shape[0], toks.data_ptr(), s)
            lg = torch.zeros(V, dtype=torch.float32, device="cuda")
            stk.decode_dev(toks.data_ptr(), n, lg.data_ptr(), graph=graph, stream=s)
            torch.cuda.synchronize()
            runs.append((toks.cpu().numpy(), lg.cpu().numpy(), dH[-1:].cpu().numpy()))
        say("flash stack tokens", runs[0][0].tolist())
        for t, l, _ in runs[1:]:
            assert np.array_equal(t, runs[0][0])
            assert np.array_equal(l.view(np.uint32), runs[0][1].view(np.uint32))
        toks = runs[0][0]
        wl, wam, _ = Z.oracle_flash(st.table, V, D, st.fnorm, st.layers[0].eps, st.softcap, F, runs[0][2])
        checks = [(wl, wam, toks[0])]
        for i in range(n):
            He = Z.oracle_embed(st.table, D, st.embed_scale, toks[i:i + 1])
            for L_, dn in zip(st.layers, st.denses):
                He = Z.oracle_block(L_, dn, He)[0]
            wl, wam, _ = Z.oracle_flash(st.table, V, D, st.fnorm, st.layers[0].eps, st.softcap, F, He)
            checks.append((wl, wam, toks[i + 1]))
        for wl, wam, tok in checks:
            fin = wl[0][np.isfinite(wl[0])]
            top2 = np.sort(fin)[-2:]
            if top2[1] - top2[0] > LOGIT_TOL:
                assert tok == wam[0], (tok, wam[0])
        # and off again: the full head's tokens
        stack.use_flash(False)
    finally:
        close_all(*objs)


def test_flash_head_every_cluster_no_forced_ids(dev):
    """FlashHead with no forced ids, and with every cluster probed: the probed ids are
    then the whole vocabulary (every id is in some cluster), and the logits are the
    full head's; both against the oracle as above."""
    table, fnorm, F, H = Z.flash_case()
    V, D = Z.FLASH_CASE["V"], Z.FLASH_CASE["D"]
    hd = zz.Head(table, V, D, fnorm, 1e-6, 1.0, 30.0)
    try:
        for NP in (F.NP, F.NC):
            F.NP, F.force = NP, np.zeros(0, np.int32)
            hd.flash(F.cent, F.NC, F.tmap, F.CS, F.NP, F.cscale, F.scaled, None)
            hd.use_flash(True)
            lg, am = hd.logits(H)
            want, wam, _ = Z.oracle_flash(table, V, D, fnorm, 1e-6, 30.0, F, H)
            fin = np.isfinite(want)
            assert np.array_equal(np.isfinite(lg), fin)
            assert float(np.abs(lg[fin] - want[fin]).max()) < LOGIT_TOL
            if NP == F.NC:
                assert fin.all()
                full, _ = Z.oracle_head(table, V, D, fnorm, 1e-6, 30.0, H)
                assert float(np.abs(lg - full).max()) < LOGIT_TOL
            for s in range(H.shape[0]):
                top2 = np.sort(want[s][fin[s]])[-2:]
                if top2[1] - top2[0] > LOGIT_TOL:
                    assert am[s] == wam[s]
    finally:
        hd.close()
