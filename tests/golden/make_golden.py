"""Write the golden vectors in tests/golden/ from the compiled reference.

Runs only where /root/reference exists and `make -C oracle` has built
oracle/_ref/libref_*.so (the reference's own q40.h / tq2.h / gemma4.c / lfm25.c /
maple.c compiled in place). Inputs are regenerated from seeds by tests/zzref.py,
so a fixture holds the case parameters, a checksum of the generated inputs and
the reference's outputs only.

    python tests/golden/make_golden.py
"""
import ctypes as C
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import zzref as Z  # noqa: E402

# (name, kind, seed, layer kwargs, S, input seed)
LAYER_CASES = [
    ("gemma_e128_s1", "gemma", 1, dict(), 1, 1),
    ("gemma_e128_s8", "gemma", 1, dict(), 8, 2),
    ("gemma_e16_s64", "gemma", 2, dict(E=16), 64, 3),
    ("lfm_q40_e32_s8", "lfm", 3, dict(fmts=(1, 1, 1)), 8, 4),
    ("lfm_q80_e32_s4", "lfm", 3, dict(fmts=(2, 2, 2)), 4, 5),
    ("maple_e256_s4", "maple", 4, dict(), 4, 6),
    ("maple_e32_s64", "maple", 4, dict(E=32), 64, 7),
]


def input_digest(L, x):
    h = hashlib.sha256()
    for a in (L.router, L.router_scale, L.pes, L.bias, L.pre_ln, L.post_ln, L.experts, x):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_cases():
    for name, kind, seed, kw, S, xseed in LAYER_CASES:
        L = Z.make_layer(kind, seed=seed, **kw)
        x = Z.make_input(L, S, xseed)
        r = Z.ref_moe(L, x)
        assert r is not None, f"reference cannot run {name}"
        np.savez(os.path.join(HERE, f"{name}.npz"), kind=kind, seed=seed, S=S, xseed=xseed,
                 kw_E=kw.get("E", -1), kw_fmts=np.array(kw.get("fmts", (0, 0, 0))),
                 digest=input_digest(L, x), out=r.out, eidx=r.eidx, ewt=r.ewt, uniq=r.uniq)
        print(name, "nu", len(r.uniq), "out rms", float(np.sqrt((r.out ** 2).mean())))


def kernel_cases():
    """Reference q4_0 / q8_0 quantiser bytes, activation quantisation and dots on a
    fixed LCG stream (the tests/test_q40.c generator, seed 12345)."""
    R = Z.ref_lib("kernels")
    R.ref_q40_dot.restype = C.c_float
    R.ref_q80_dot.restype = C.c_float
    R.ref_tq2_dot.restype = C.c_float
    R.ref_tq2_quant_act.restype = C.c_float
    rs = np.uint32(12345)
    vals = np.empty(1 << 17, np.float32)
    for i in range(vals.size):   # rs = rs*1664525 + 1013904223; (rs>>8)/2^23 - 1
        rs = np.uint32((int(rs) * 1664525 + 1013904223) & 0xffffffff)
        vals[i] = np.float32(np.float32(int(rs) >> 8) / np.float32(8388608.0) - np.float32(1.0))
    O, I = 16, 2816
    w = (vals[:O * I] * np.float32(0.1)).astype(np.float32)
    q40 = np.zeros(O * I // 32 * 18, np.uint8)
    q80 = np.zeros(O * I // 32 * 34, np.uint8)
    R.ref_q40_quant_row(Z.ptr(w), Z.ptr(q40), O * I)
    R.ref_q80_quant_row(Z.ptr(w), Z.ptr(q80), O * I)
    x = vals[O * I:O * I + 4 * I].reshape(4, I).copy()
    x[1] *= np.float32(37.0)
    x[2, :64] = 0.0                                  # all-zero blocks: d = 0, q = 0
    xq = np.zeros((4, I), np.int8)
    xs = np.zeros((4, I // 32), np.float32)
    for t in range(4):
        R.ref_quant_act(Z.ptr(x[t]), Z.ptr(xq[t]), Z.ptr(xs[t]), I)
    d40 = np.zeros((4, O), np.float32)
    d80 = np.zeros((4, O), np.float32)
    for t in range(4):
        for o in range(O):
            d40[t, o] = R.ref_q40_dot(Z.ptr(q40[o * (I // 32) * 18:]), Z.ptr(xq[t]), Z.ptr(xs[t]), I)
            d80[t, o] = R.ref_q80_dot(Z.ptr(q80[o * (I // 32) * 34:]), Z.ptr(xq[t]), Z.ptr(xs[t]), I)
    # tq2 at the Maple shape, rows of the LCG mapped to codes 0,1,2
    It = 2048
    codes = (np.abs((vals[:O * It] * 3).astype(np.int32)) % 3).astype(np.int8).reshape(O, It)
    alpha = (np.abs(vals[-O:]) * np.float32(0.03) + np.float32(0.001)).astype(np.float32)
    tq = Z.tq2_tensor(codes, alpha)
    xt = vals[:It].copy()
    tq_q = np.zeros(It, np.int8)
    tq_s = np.zeros(It // 32, np.float32)
    tot = R.ref_tq2_quant_act(Z.ptr(xt), Z.ptr(tq_q), Z.ptr(tq_s), It)
    dtq = np.zeros(O, np.float32)
    cb = tq[O * 4:]
    for o in range(O):
        dtq[o] = R.ref_tq2_dot(Z.ptr(cb[o * (It // 4):]), C.c_float(alpha[o]), Z.ptr(tq_q),
                               Z.ptr(tq_s), C.c_float(tot), It)
    # the exact-activation dots (q40.h:290-305, 443-455, tq2.h:235-252) on the same
    # rows and the unquantised x
    for n in ("ref_q40_dot_f32", "ref_q80_dot_f32", "ref_tq2_dot_f32"):
        getattr(R, n).restype = C.c_float
    d40f = np.zeros((4, O), np.float32)
    d80f = np.zeros((4, O), np.float32)
    for t in range(4):
        xt_ = np.ascontiguousarray(x[t])
        for o in range(O):
            d40f[t, o] = R.ref_q40_dot_f32(Z.ptr(q40[o * (I // 32) * 18:]), Z.ptr(xt_), I)
            d80f[t, o] = R.ref_q80_dot_f32(Z.ptr(q80[o * (I // 32) * 34:]), Z.ptr(xt_), I)
    dtqf = np.zeros(O, np.float32)
    for o in range(O):
        dtqf[o] = R.ref_tq2_dot_f32(Z.ptr(cb[o * (It // 4):]), C.c_float(alpha[o]), Z.ptr(xt), It)
    # q4a (tq2.h:269-292, 405-427): nibble bytes from the LCG's mantissas, d and m in
    # maple.c:1790-1796's ranges, against the same four x rows
    R.ref_q4a_dot_f32.restype = C.c_float
    R.ref_f32_to_fp16.restype = C.c_uint16
    ng = O * (I // 64)
    q4a = np.zeros((ng, 36), np.uint8)
    bits = (vals.view(np.uint32)[:ng * 32] >> np.uint32(7)).astype(np.uint8)
    q4a[:, 4:] = bits.reshape(ng, 32)
    for g in range(ng):
        hd = R.ref_f32_to_fp16(C.c_float(0.002 + 0.01 * abs(float(vals[-1 - g]))))
        hm = R.ref_f32_to_fp16(C.c_float(0.05 * float(vals[-1 - ng - g])))
        q4a[g, :4] = [hd & 255, hd >> 8, hm & 255, hm >> 8]
    q4a = q4a.reshape(-1)
    dq4af = np.zeros((4, O), np.float32)
    for t in range(4):
        xt_ = np.ascontiguousarray(x[t])
        for o in range(O):
            dq4af[t, o] = R.ref_q4a_dot_f32(Z.ptr(q4a[o * (I // 64) * 36:]), Z.ptr(xt_), I)
    np.savez(os.path.join(HERE, "kernels_lcg12345.npz"), w=w, q40=q40, q80=q80, x=x, xq=xq,
             xs=xs, d40=d40, d80=d80, codes=codes, alpha=alpha, tq=tq, xt=xt, tq_q=tq_q,
             tq_s=tq_s, tq_tot=np.float32(tot), dtq=dtq, d40f=d40f, d80f=d80f, dtqf=dtqf,
             q4a=q4a, dq4af=dq4af)
    print("kernels_lcg12345: q40", q40.nbytes, "B, dots", d40.size + d80.size + dtq.size,
          "f32 dots", d40f.size + d80f.size + dtqf.size + dq4af.size)


def gemma_cases():
    """The feed-forward half of layer_fwd, embed_row, the tied head with greedy
    selection, and a two-layer stack's prefill + greedy decode, from the compiled
    reference (gemma4.c:1003-1030, 1131-1145, 1264-1275, 2149-2152)."""
    L, dn, H, table, fnorm, st, H0 = Z.gemma_block_case()
    D, MI, E, K, DI, V, seed = Z.GEMMA_SHAPE
    Hb, eidx, ewt = Z.ref_block(L, dn, H)
    emb = Z.ref_embed(table, V, D, np.float32(np.sqrt(np.float32(D))), Z.GEMMA_TOKS)
    lg, am = Z.ref_head(table, V, D, fnorm, L.eps, 30.0, H[:3])
    toks, Hp, lg_last = Z.ref_stack(st, H0, Z.GEMMA_STACK["steps"])
    np.savez(os.path.join(HERE, "gemma_block_stack.npz"), digest=Z.gemma_digest(L, dn, H, table, fnorm, st, H0),
             block_H=Hb, block_eidx=eidx, block_ewt=ewt, embed=emb, head_logits=lg, head_argmax=am,
             stack_tokens=toks, stack_prefill=Hp, stack_logits=lg_last)
    print("gemma_block_stack: tokens", toks.tolist(), "head argmax", am.tolist())


def flash_cases():
    """FlashHead (gemma4.c:1055-1131 + sample at temp 0) from the compiled reference:
    the plain case and the all-ties case of zzref.flash_case. The chosen clusters are
    read off the logits: those whose members all came out finite."""
    f = Z.FLASH_CASE
    out = {}
    for key, (scaled, tie_all) in (("plain", (1, False)), ("ties", (1, True))):
        table, fnorm, F, H = Z.flash_case(scaled, tie_all)
        lg, am = Z.ref_flash(table, f["V"], f["D"], fnorm, 1e-6, 30.0, F, H)
        fin = np.isfinite(lg)
        sel = np.array([[c for c in range(F.NC) if (F.tmap[c] >= 0).any() and fin[s][F.tmap[c][F.tmap[c] >= 0]].all()]
                        for s in range(H.shape[0])], np.int32)
        out.update({f"{key}_argmax": am, f"{key}_sel": sel, f"{key}_finite": fin,
                    f"{key}_logits": lg[fin]})
        print("gemma_flash_head", key, "argmax", am.tolist(), "clusters", sel[0].tolist())
    np.savez(os.path.join(HERE, "gemma_flash_head.npz"), **out)


def zipf_cases():
    """configs[1]'s Zipf-offset router at the Gemma-4 shape. The reference router has
    no offset (gemma4.c:600-601); zzref.zipf_pin_case carries it in the reference
    layer's last router column, whose product is exactly the offset, so the
    reference computes fl(chain + offset) as the configs[1] harness defines it."""
    c = dict(Z.ZIPF_PIN)
    Lo, Lr, x = Z.zipf_pin_case(**c)
    r = Z.ref_moe(Lr, x)
    np.savez(os.path.join(HERE, "gemma_zipf_e128_s8.npz"), digest=input_digest(Lr, x),
             out=r.out, eidx=r.eidx, ewt=r.ewt, uniq=r.uniq, **{f"case_{k}": v for k, v in c.items()})
    print("gemma_zipf_e128_s8 nu", len(r.uniq), "ids", r.eidx[:8].tolist())


ALL = dict(kernels=kernel_cases, layers=layer_cases, gemma=gemma_cases, flash=flash_cases,
           zipf=zipf_cases)

if __name__ == "__main__":
    if Z.ref_lib("gemma4") is None:
        sys.exit("oracle/_ref is not built (needs /root/reference): run `make -C oracle`")
    for name in (sys.argv[1:] or list(ALL)):      # e.g. `make_golden.py zipf`
        ALL[name]()
