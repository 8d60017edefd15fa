"""Build libzzmoe.so (the HIP library behind include/zz_gpu.h and include/zz_moe.h)
for gfx950 with hipcc, in-tree, plus the C host harness that mirrors the engines'
moe_start/moe_finish boundary.

    python -m zunzuncito_amd.build          # or: python zunzuncito_amd/build.py
"""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libzzmoe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["zz_api.hip", "zz_route.hip", "zz_ffn.hip", "zz_matmul.hip", "zz_quant.hip", "zz_mma_up.hip", "zz_mma_down.hip", "zz_decode.hip",
           "zz_gemma.hip", "zz_container.hip", "zz_flash.hip"]

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # every fused multiply-add is explicit (fmaf) so bit-level behaviour is chosen
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # no packed-fp32 instructions from the compiler
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core results straight into VGPRs (no v_accvgpr_read per element)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed: {what}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise
    return [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]


def build(verbose=True, jobs=None):
    """Each source to an object in parallel (into _build/, git-ignored), then one
    shared library."""
    from concurrent.futures import ThreadPoolExecutor
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    odir = os.path.join(PKG, "_build")
    os.makedirs(odir, exist_ok=True)
    objs = [os.path.join(odir, os.path.basename(s) + ".o") for s in srcs]
    cflags = [f for f in FLAGS if f != "-shared"] + ["-I", os.path.join(ROOT, "include"), "-c"]
    if verbose:
        print(" ".join([HIPCC] + cflags + ["<src>", "-o", "<obj>"]), flush=True)
    jobs = jobs or min(len(srcs), os.cpu_count() or 4)
    with ThreadPoolExecutor(jobs) as ex:
        notes = list(ex.map(lambda so: _run([HIPCC] + cflags + [so[0], "-o", so[1]], so[0]), zip(srcs, objs)))
    tmp = LIB + ".tmp"
    notes.append(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, "link"))
    noise = [ln for n in notes for ln in n]
    if noise and verbose:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
