"""BASELINE configs[4] at its size: the Gemma-4-shaped stack of 30 layers x 128 q4_0
experts (12.8 GB resident in HBM) with a q4_0 dense MLP per layer and the tied
262144-row head, attention the identity, a 512-token prefill and 256 greedy decode
steps: gemma4.c forward() (1184-1276) with the layers' attention skipped, its FFN
half 998-1030. The stack is built by bench.py's own generator, so this is the
workload the benchmark times.

  - the stack's prefill equals the 30 blocks run one by one, bit for bit, and its
    greedy token is the head's argmax of the last row;
  - 256 greedy steps replayed from a captured HIP graph equal eager launches bit
    for bit (tokens and last logits), and the first steps equal the blocks, embed
    and head run one by one;
  - layers 0 and 29 at S = 512, and every layer in the first decode step, against
    the CPU oracle on the GPU's own input to that layer (so differences cannot
    cascade): routing ids exact, outputs within the fp32 tier.
"""
import sys

import numpy as np
import pytest

import bench
import zzref as Z
import zunzuncito_amd as zz

pytestmark = pytest.mark.gpu

SEED = 1                 # bench.py's default --seed
NL, S, STEPS = 30, 512, 256
OUT_TOL = 1e-3
LOGIT_TOL = 1e-3         # head logits, absolute (softcapped at 30), as tests/test_gpu_gemma.py


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def c5():
    import torch
    zz.init()
    say("config 5: building 30 layers x 128 experts, dense MLPs and the head")
    layers, host = bench.build_layers(zz, torch, NL, SEED)
    c = bench.build_stack(zz, torch, layers, SEED, flash=False, keep_host=True)
    c["layers"], c["host"] = layers, host
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED + 99)
    c["H0"] = torch.randn(S, bench.D, generator=g, device="cuda")        # bench.py's prefill rows
    # the blocks one by one, keeping every layer's input and the routing of 0 and 29
    st = torch.cuda.current_stream().cuda_stream
    h = c["H0"].clone()
    c["ins"], c["ids"] = {}, {}
    for l, B in enumerate(c["blocks"]):
        if l in (0, NL - 1):
            c["ins"][l] = h.cpu().numpy()
            ix = torch.zeros(S * bench.K, dtype=torch.int32, device="cuda")
            B.forward_dev(h.data_ptr(), S, d_eidx=ix.data_ptr(), stream=st)
            c["ids"][l] = (ix, h.clone())
        else:
            B.forward_dev(h.data_ptr(), S, stream=st)
    torch.cuda.synchronize()
    c["bb"] = h
    say("config 5 built")
    yield c
    for o in c["objs"]:
        o.close()
    for m in layers:
        m.close()


def oracle_layer(c, l, ids=None):
    """zzref's Layer and Dense of block l (experts regenerated on the device; only
    `ids` when given), for orc_gemma_ffn_block."""
    import torch
    h = c["host"][l]
    L_ = Z.Layer(bench.D, bench.MI, bench.E, bench.K, Z.GATE_GEMMA, Z.ACT_GEGLU_TANH, (1, 1, 1), eps=1e-6)
    L_.router, L_.router_scale, L_.pes = h["router"], h["rscale"], h["pes"]
    L_.bias, L_.use_bias = h["zipf"], 1
    L_.pre_ln, L_.post_ln = h["pre"], h["post"]
    L_.experts = bench.layer_experts_host(zz, torch, SEED, l, ids)
    L_.esz = bench.REC_B
    d = c["dense"][l]
    dn = Z.Dense(bench.D, bench.DI, d["mlp"], d["pre_ffn_ln"], d["post_ffn_ln1"], d["post_ffn_ln"],
                 d["layer_scalar"])
    return L_, dn


def test_config5_prefill_equals_blocks(c5):
    import torch
    st = torch.cuda.current_stream().cuda_stream
    a = c5["H0"].clone()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    say("config 5: stack prefill of 512 rows")
    c5["stack"].prefill_dev(a.data_ptr(), S, tok.data_ptr(), st)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), c5["bb"].view(torch.int32))
    # the prefill's greedy token: the head's argmax of the last row
    lg = torch.zeros(bench.V, dtype=torch.float32, device="cuda")
    t2 = torch.zeros(1, dtype=torch.int32, device="cuda")
    last = c5["bb"][-1:].clone()
    c5["head"].logits_dev(last.data_ptr(), 1, lg.data_ptr(), t2.data_ptr(), st)
    torch.cuda.synchronize()
    assert int(tok.item()) == int(t2.item()) == int(torch.argmax(lg).item())
    c5["tok0"] = int(tok.item())


def test_config5_decode_graph_equals_eager(c5):
    import torch
    st = torch.cuda.current_stream().cuda_stream
    tok0 = c5.get("tok0", 0)
    runs = []
    for graph in (False, True, True):
        say(f"config 5: {STEPS} greedy steps, graph={graph}")
        toks = torch.zeros(STEPS + 1, dtype=torch.int32, device="cuda")
        toks[0] = tok0
        lg = torch.zeros(bench.V, dtype=torch.float32, device="cuda")
        c5["stack"].decode_dev(toks.data_ptr(), STEPS, lg.data_ptr(), graph=graph, stream=st)
        torch.cuda.synchronize()
        runs.append((toks.cpu().numpy(), lg.cpu().numpy()))
        junk = torch.randn(4096, device="cuda")                    # eager work between replays
        assert float(junk.abs().sum()) > 0
    for t, l in runs[1:]:
        assert np.array_equal(t, runs[0][0])
        assert np.array_equal(l.view(np.uint32), runs[0][1].view(np.uint32))
    say("  distinct tokens", len(np.unique(runs[0][0])), "first", runs[0][0][:12].tolist())
    # the first steps with the blocks, embed and head run one by one (each block's
    # combine in its own kernel instead of deferred into the next block's router)
    n = 3
    h1 = torch.zeros((1, bench.D), dtype=torch.float32, device="cuda")
    dl = torch.zeros((1, bench.V), dtype=torch.float32, device="cuda")
    dtok = torch.tensor([tok0], dtype=torch.int32, device="cuda")
    man = [tok0]
    for _ in range(n):
        c5["head"].embed_dev(dtok.data_ptr(), 1, h1.data_ptr(), st)
        for B in c5["blocks"]:
            B.forward_dev(h1.data_ptr(), 1, stream=st)
        c5["head"].logits_dev(h1.data_ptr(), 1, dl.data_ptr(), dtok.data_ptr(), st)
        man.append(int(dtok.item()))
    assert man == runs[0][0][:n + 1].tolist(), (man, runs[0][0][:n + 1])
    c5["toks"] = runs[0][0]


@pytest.mark.parametrize("l", [0, NL - 1])
def test_config5_prefill_layer_vs_oracle(c5, l):
    """Layer l at S = 512 on the GPU's own input to it."""
    Z.oracle().orc_set_threads(16)
    L_, dn = oracle_layer(c5, l)
    H_in = c5["ins"][l]
    say(f"config 5: layer {l} at S=512 against the oracle")
    Hw, eidx, ewt = Z.oracle_block(L_, dn, H_in)
    ix, hout = c5["ids"][l]
    got_ids, got = ix.cpu().numpy(), hout.cpu().numpy()
    assert np.array_equal(got_ids, eidx), int((got_ids != eidx).sum())
    sc = np.float32(dn.layer_scalar)
    err = Z.rel_l2(got, Hw)
    err_ffn = Z.rel_l2(got - H_in * sc, Hw - H_in * sc)         # the FFN half alone
    say(f"  ids exact, rel L2 {err:.2e}, FFN half {err_ffn:.2e}")
    assert err < OUT_TOL and err_ffn < OUT_TOL


def test_config5_decode_step_every_layer_vs_oracle(c5):
    """The first decode step through all 30 layers, each layer on the GPU's own
    input: ids exact and the block output within the fp32 tier."""
    import torch
    st = torch.cuda.current_stream().cuda_stream
    Z.oracle().orc_set_threads(16)
    tok0 = c5.get("tok0", 0)
    h = torch.zeros((1, bench.D), dtype=torch.float32, device="cuda")
    dtok = torch.tensor([tok0], dtype=torch.int32, device="cuda")
    c5["head"].embed_dev(dtok.data_ptr(), 1, h.data_ptr(), st)
    worst = 0.0
    for l, B in enumerate(c5["blocks"]):
        H_in = h.cpu().numpy()
        ix = torch.zeros(bench.K, dtype=torch.int32, device="cuda")
        B.forward_dev(h.data_ptr(), 1, d_eidx=ix.data_ptr(), stream=st)
        got_ids, got = ix.cpu().numpy(), h.cpu().numpy()
        L_, dn = oracle_layer(c5, l, ids=got_ids)
        Hw, eidx, _ = Z.oracle_block(L_, dn, H_in)
        assert np.array_equal(got_ids, eidx), (l, got_ids, eidx)
        sc = np.float32(dn.layer_scalar)
        err = max(Z.rel_l2(got, Hw), Z.rel_l2(got - H_in * sc, Hw - H_in * sc))
        worst = max(worst, err)
        assert err < OUT_TOL, (l, err)
    say(f"config 5: decode step, 30 layers: ids exact, worst rel L2 {worst:.2e}")
    # the head on the last layer's output: logits and the greedy token
    lg = torch.zeros((1, bench.V), dtype=torch.float32, device="cuda")
    t1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    H_last = h.cpu().numpy()
    c5["head"].logits_dev(h.data_ptr(), 1, lg.data_ptr(), t1.data_ptr(), st)
    wl, wam = Z.oracle_head(c5["table"], bench.V, bench.D, c5["fnorm"], 1e-6, 30.0, H_last)
    d = float(np.abs(lg.cpu().numpy() - wl).max())
    top2 = np.sort(wl[0])[-2:]
    say(f"  head: max |logit diff| {d:.2e}, token {int(t1.item())}, oracle {int(wam[0])}")
    assert d < LOGIT_TOL
    if top2[1] - top2[0] > LOGIT_TOL:
        assert int(t1.item()) == int(wam[0])
    if "toks" in c5:                        # the decode run's first greedy token
        assert int(c5["toks"][1]) == int(t1.item())
