"""An engine-shaped C caller (tests/engine_harness.c) against libzzmoe.so: the layer is
registered at load like an engine's slot fill, the forward goes through moe_start /
moe_finish patched the way gemma4.c:750 / 792 would be, and the CPU path stands in
for the engine's own when the library declines. Also the reference engines themselves,
built against libzzmoe.so in place of their Metal backend (oracle/Makefile), running
their own --check-gpu (gemma4.c:2315-2368, lfm25.c, maple.c:1756-1826, ling.c)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import zzref as Z

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
HARNESS = os.path.join(HERE, "_bin", "engine_harness")
ENGINES = ("gemma4", "lfm25", "maple", "ling")


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def write_case(path, L, x):
    """case.bin in the layout engine_harness.c reads."""
    S = x.shape[0]
    hdr = np.array([L.D, L.MI, L.E, L.K, L.gating, L.act, *L.fmts, L.norm_topk, L.use_bias,
                    L.n_group, L.topk_group, S, L.router_scale is not None, L.pes is not None,
                    L.bias is not None, L.pre_ln is not None], np.int32)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.array([L.eps, L.routed_scaling, L.clamp], np.float32).tobytes())
        f.write(np.array([L.esz], np.int64).tobytes())
        for a in (L.router, L.router_scale, L.pes, L.bias, L.pre_ln, L.post_ln):
            if a is not None:
                f.write(np.ascontiguousarray(a, np.float32).tobytes())
        f.write(np.ascontiguousarray(L.experts, np.uint8).tobytes())
        f.write(np.ascontiguousarray(x, np.float32).tobytes())


def run_harness(tmp_path, L, x, env=None):
    if not os.path.exists(HARNESS):
        pytest.skip("tests/_bin/engine_harness not built (make -C tests)")
    case, res = tmp_path / "case.bin", tmp_path / "result.bin"
    write_case(case, L, x)
    p = subprocess.run([HARNESS, str(case), str(res)], capture_output=True, text=True,
                       timeout=300, env={**os.environ, **(env or {})})
    say(p.stdout.strip(), p.stderr.strip())
    assert p.returncode == 0, (p.returncode, p.stdout, p.stderr)
    S = x.shape[0]
    r = np.fromfile(res, np.uint8)
    nd, nk = S * L.D * 4, S * L.K * 4
    assert r.size == nd + 2 * nk
    out = r[:nd].view(np.float32).reshape(S, L.D)
    eidx = r[nd:nd + nk].view(np.int32)
    ewt = r[nd + nk:].view(np.float32)
    path = p.stdout.split("path ")[1].split()[0]
    assert "declines ok" in p.stdout
    return path, out, eidx, ewt


CASES = [("gemma", 5), ("lfm", 16), ("maple", 3), ("ling", 9)]


def small(kind):
    L = Z.make_layer(kind, seed=21, K=4, D=512, MI=256, E=16)
    if kind == "ling":
        L.n_group, L.topk_group = 4, 2
    return L


@pytest.mark.parametrize("kind,S", CASES)
def test_harness_cpu_path(tmp_path, kind, S):
    """With the library declining (ZZ_DISABLE=1, or no GPU), the engine's CPU path runs
    and its result is the CPU restatement's, bit for bit."""
    L = small(kind)
    x = Z.make_input(L, S, 31)
    path, out, eidx, ewt = run_harness(tmp_path, L, x, {"ZZ_DISABLE": "1"})
    assert path == "cpu"
    want = Z.oracle_moe(L, x)
    assert np.array_equal(eidx, want.eidx)
    assert np.array_equal(out.view(np.uint32), want.out.view(np.uint32))
    assert np.array_equal(ewt.view(np.uint32), want.ewt.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("kind,S", CASES)
def test_harness_gpu_path(tmp_path, kind, S):
    """The same engine-shaped caller on the GPU: the routing equals the CPU path's
    exactly and the output is within the layer tolerance."""
    L = small(kind)
    x = Z.make_input(L, S, 31)
    say(f"harness {kind} S={S}")
    path, out, eidx, ewt = run_harness(tmp_path, L, x)
    assert path == "gpu"
    want = Z.oracle_moe(L, x)
    assert np.array_equal(eidx, want.eidx)
    np.testing.assert_allclose(ewt, want.ewt, rtol=1e-4, atol=1e-6)
    assert Z.rel_l2(out, want.out) < 1e-3


def _engine(name):
    exe = os.path.join(REPO, "oracle", "_ref", f"{name}_zz")
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (needs the reference sources)")
    return exe


@pytest.mark.parametrize("name", ENGINES)
def test_reference_engine_without_device(tmp_path, name):
    """Linked against libzzmoe.so with the library declining, each engine's own
    --check-gpu reports that there is nothing to check and exits 0."""
    p = subprocess.run([_engine(name), str(tmp_path / "none"), "--check-gpu"], capture_output=True,
                       text=True, timeout=120, env={**os.environ, "ZZ_DISABLE": "1"})
    say(p.stdout.strip())
    assert p.returncode == 0 and "nothing to check" in p.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("name", ENGINES)
def test_reference_engine_check_gpu(tmp_path, name):
    """Each reference engine's own --check-gpu, unchanged, through libzzmoe.so's
    gpu.h entry points on the MI355X."""
    say(f"engine {name} --check-gpu")
    p = subprocess.run([_engine(name), str(tmp_path / "none"), "--check-gpu"], capture_output=True,
                       text=True, timeout=300)
    say(p.stdout.strip(), p.stderr.strip()[-2000:])
    assert p.returncode == 0, p.stdout
    assert "GPU CHECK PASSED" in p.stdout
