"""zz_expf (zunzuncito_amd/csrc/zz_expf.h), the expf the sigmoid routers use on the
device, against the host libm's expf (glibc, the reference's: lfm25.c:654,
ling.c:731) on every one of the 2^32 float inputs, bit for bit. tests/expf_check.hip
is compiled for the host with hipcc and makes no GPU call."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-fopenmp", "-ffp-contract=off",
                    os.path.join(HERE, "expf_check.hip"), "-o", exe], check=True, capture_output=True)
    return exe


def test_zz_expf_equals_host_expf_on_all_floats(checker):
    r = subprocess.run([checker], capture_output=True, text=True, timeout=600)
    print(r.stdout.strip())
    assert r.returncode == 0 and " mismatches 0 " in r.stdout, r.stdout + r.stderr
