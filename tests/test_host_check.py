"""The host-only code of the library -- the container manifest parser and the gpu_map
range registry (zunzuncito_amd/csrc/zz_manifest.h) -- checked by tests/host_check.cpp,
built plain and under AddressSanitizer + UndefinedBehaviorSanitizer (tests/Makefile):
valid gemma / maple (esz) and lfm / ling (eszl) manifests, values that cannot be sizes
or indices, over-long lines, a missing file, 3000 random manifests, and ranges nested,
touching and at the top of the address space."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("name", ["host_check", "host_check_san"])
def test_host_check(tmp_path, name):
    exe = os.path.join(HERE, "_bin", name)
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (make -C tests)")
    # the sanitizer runtime must come first; a preload that a harness adds is tolerated
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    p = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=300, env=env)
    assert p.returncode == 0, p.stdout + p.stderr[-3000:]
    assert "host_check ok" in p.stdout
