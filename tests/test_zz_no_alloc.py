"""zz_moe_forward_dev_noalloc: the device-pointer forward on the library's fixed
scratch array. Checked against zz_moe_forward_dev (the entry point it mirrors) on
three calls in a row, each smaller (matrix-core path, then two decode batches), bit
for bit, and against the oracle at the
parity bar (ids exact, rel L2 < 1e-3); a batch beyond the scratch is declined with
its outputs untouched."""
import sys

import numpy as np
import pytest

import zzref as Z
import zunzuncito_amd as zz

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def test_noalloc_forward_equals_forward_dev():
    import torch
    zz.init()
    L = Z.make_layer("gemma", seed=21, E=32, zipf=True)
    m = zz.MoeLayer(L.D, L.MI, L.E, L.K, L.gating, L.act, L.fmts, L.router, L.router_scale,
                    L.pes, L.bias, L.pre_ln, L.post_ln, use_bias=L.use_bias, eps=L.eps)
    try:
        m.upload_all(L.experts)
        s = torch.cuda.current_stream().cuda_stream
        # each call smaller than the last: the matrix-core path, then the decode path
        # (S <= 2 for q4_0 layers) twice, all on the same scratch array
        for S in (200, 2, 1):
            say(f"noalloc vs forward_dev: gemma E=32, S={S}")
            x = Z.make_input(L, S, 40 + S)
            din = torch.from_numpy(x).cuda()
            outs = []
            for noalloc in (False, True):
                dout = torch.full((S, L.D), float("nan"), dtype=torch.float32, device="cuda")
                dix = torch.full((S * L.K,), -1, dtype=torch.int32, device="cuda")
                dwt = torch.zeros(S * L.K, dtype=torch.float32, device="cuda")
                args = (din.data_ptr(), dout.data_ptr(), S, dix.data_ptr(), dwt.data_ptr(), s)
                if noalloc:
                    assert m.forward_dev_noalloc(*args), zz.last_error()
                else:
                    m.forward_dev(*args)
                torch.cuda.synchronize()
                outs.append((dout.cpu().numpy(), dix.cpu().numpy(), dwt.cpu().numpy()))
            (o0, i0, w0), (o1, i1, w1) = outs
            assert np.array_equal(i1, i0) and np.array_equal(w1.view(np.uint32), w0.view(np.uint32))
            assert np.array_equal(o1.view(np.uint32), o0.view(np.uint32))
            want = Z.oracle_moe(L, x)
            err = Z.rel_l2(o1, want.out)
            say(f"  ids exact {np.array_equal(i1, want.eidx)}, rel L2 vs oracle {err:.2e}")
            assert np.array_equal(i1, want.eidx) and err < 1e-3
        # a chunk whose workspace exceeds the scratch: declined, outputs untouched
        S = 1024
        din = torch.zeros((S, L.D), dtype=torch.float32, device="cuda")
        dout = torch.full((S, L.D), 7.0, dtype=torch.float32, device="cuda")
        assert not m.forward_dev_noalloc(din.data_ptr(), dout.data_ptr(), S, 0, 0, s)
        assert "scratch" in zz.last_error()
        torch.cuda.synchronize()
        assert bool((dout == 7.0).all())
    finally:
        m.close()
