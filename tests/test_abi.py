"""The C-ABI library loads, exports exactly what include/*.h declares, and honours
the decline contract when no GPU is present (gpu.h:31-33, 90-107): every call
returns 0 (or -1 for a layer id) and leaves its outputs untouched."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import zunzuncito_amd as zz

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:gpu|zz)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_headers_and_binding_agree():
    assert declared_symbols() == set(zz.ABI_SYMBOLS)


def test_library_exports_every_declared_symbol():
    zz.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", zz.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = declared_symbols() - exported
    assert not missing, missing


def test_headers_compile_as_c():
    src = '#include "zz_gemma.h"\nint main(void){ return gpu_ready(); }\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I",
                        os.path.join(ROOT, "include"), "-x", "c", "-"], input=src,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _has_gpu():
    r = subprocess.run(["python", "-c", "import zunzuncito_amd as z; import sys; "
                        "sys.exit(0 if z.lib().gpu_init() else 1)"], capture_output=True)
    return r.returncode == 0


@pytest.mark.skipif(os.environ.get("ZZ_ASSUME_GPU") == "1", reason="GPU box")
def test_decline_contract_without_device():
    if _has_gpu():
        pytest.skip("a gfx950 device is present: the decline path is not reachable")
    L = zz.lib()
    assert L.gpu_init() == 0
    assert zz.last_error()
    assert L.gpu_ready() == 0
    assert L.gpu_name() == b"none"
    w = np.zeros(4096, np.uint8)
    assert L.gpu_map(C.c_void_p(w.ctypes.data), w.nbytes) == 0
    x = np.ones((1, 64), np.float32)
    y = np.full((1, 8), 7.0, np.float32)
    assert L.gpu_q40_matmul(y.ctypes.data_as(zz._f32p), w.ctypes.data_as(zz._u8p),
                            x.ctypes.data_as(zz._f32p), 8, 64, 1) == 0
    assert np.all(y == 7.0)                      # outputs untouched on decline
    d = zz.ZzMoeDesc(64, 64, 4, 2, 0, 0, 1, 1, 1, 1, 0, 1e-6, 1.0, 7.0)
    r = np.zeros(256, np.float32)
    wts = zz.ZzMoeWeights(r.ctypes.data_as(zz._f32p), None, None, None, None, None)
    assert L.zz_moe_layer_create(C.byref(d), C.byref(wts)) == -1
    out = np.full((1, 64), 3.0, np.float32)
    assert L.zz_moe_forward(0, x.ctypes.data_as(zz._f32p), out.ctypes.data_as(zz._f32p), 1,
                            None, None) == 0
    assert np.all(out == 3.0)
    assert L.zz_moe_stats((C.c_uint * 4)()) == 0
    ln = np.ones(64, np.float32)
    assert L.zz_ffn_block_create(0, 1, ln.ctypes.data_as(zz._f32p), 1.0) == -1
    assert L.zz_ffn_block_forward(0, out.ctypes.data_as(zz._f32p), 1, None, None) == 0
    assert np.all(out == 3.0)
    tab = np.zeros(64 * 2 * 18, np.uint8)
    assert L.zz_head_create(tab.ctypes.data_as(zz._u8p), 64, 64, ln.ctypes.data_as(zz._f32p),
                            1e-6, 8.0, 30.0) == -1
    tok = np.zeros(1, np.int32)
    assert L.zz_head_embed(0, tok.ctypes.data_as(zz._i32p), 1, out.ctypes.data_as(zz._f32p)) == 0
    lg = np.full((1, 64), 5.0, np.float32)
    assert L.zz_head_logits(0, x.ctypes.data_as(zz._f32p), 1, lg.ctypes.data_as(zz._f32p),
                            tok.ctypes.data_as(zz._i32p)) == 0
    assert np.all(out == 3.0) and np.all(lg == 5.0)
    ids = np.zeros(2, np.int32)
    assert L.zz_stack_create(ids.ctypes.data_as(zz._i32p), 2, 0) == -1
    assert L.zz_stack_decode_dev(0, None, 4, None, 1, None) == 0
    assert L.zz_moe_load_experts(0, b"/nonexistent", 0) == 0
    assert L.zz_gemma_stack_load(b"/nonexistent", None, None, None) == -1
    L.gpu_shutdown()                             # safe when never initialised


def test_record_bytes_match_reference_sizes():
    """zz_moe_record_bytes = the reference record [gate|up|down] (q40.h:313-314,
    461-462; tq2.h:84-86) for every BASELINE shape."""
    L = zz.lib()
    cases = [((2816, 704, 128, 8, 0, 0, 1, 1, 1), 3 * 1115136),
             ((2048, 1792, 32, 4, 1, 1, 1, 1, 2), 2 * 2064384 + 3899392),
             ((2048, 768, 256, 8, 2, 2, 3, 3, 3), 2 * 396288 + 401408)]
    for args, want in cases:
        d = zz.ZzMoeDesc(*args, 1, 0, 1e-6, 1.0, 7.0)
        assert L.zz_moe_record_bytes(C.byref(d)) == want
    bad = zz.ZzMoeDesc(2816, 700, 128, 8, 0, 0, 1, 1, 1, 1, 0, 1e-6, 1.0, 7.0)   # MI % 64
    assert L.zz_moe_record_bytes(C.byref(bad)) == -1
