"""The byte and operation accounting behind bench.py's roofline and matrix-core
figures, and the profile lines it reads (CPU only; nothing here touches a GPU)."""
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def test_q40_tensor_bytes():
    # gemma4.c's expert: gate and up [704 x 2816], down [2816 x 704], 18 bytes per
    # 32-weight block (fp16 scale + 16 nibble bytes)
    assert bench.tensor_bytes(1, 704, 2816) == 704 * 88 * 18 == 1115136
    assert bench.rec_bytes(bench.CONFIGS["gemma"]) == 3 * 1115136
    # q8_0: 34 bytes per block
    assert bench.tensor_bytes(2, 2048, 1792) == 2048 * 56 * 34


def test_algorithmic_bytes_gemma_s512():
    c = bench.CONFIGS["gemma"]
    nu, S = 91.0, 512
    by = bench.algorithmic_bytes(c, S, nu)
    P = S * 8
    xq = S * 2816 + S * 88 * 8                  # int8 codes + f32 scale and int sum per block
    h = P * 704 + P * 22 * 8
    assert by["ffn_up"] == nu * 2 * 1115136 + xq + h
    assert by["ffn_down"] == nu * 1115136 + h + P * 2816 * 4
    # the layer counts each expert tensor once, plus router, norms, input and output
    assert by["layer"] == nu * 3 * 1115136 + 128 * 2816 * 4 + 3 * 2816 * 4 + 128 * 8 + 2 * S * 2816 * 4


def test_mfma_use_counts_useful_int8_operations():
    c = bench.CONFIGS["gemma"]
    m = bench.mfma_use(c, 512, {"ffn_up": 100.0, "ffn_down": 50.0, "prep": 9.0}, "gemma512")
    up_ops = 2.0 * 4096 * 2 * 704 * 2816        # gate and up, 2 operations per multiply-add
    assert m["ffn_up"]["int8_ops"] == up_ops
    assert m["ffn_up"]["achieved"] == pytest.approx(up_ops / 100e-6 / 1e12)
    assert m["ffn_up"]["frac"] == pytest.approx(m["ffn_up"]["achieved"] / 5000.0)
    assert m["ffn_down"]["int8_ops"] == up_ops / 2
    # the decode path runs dot4 GEMV kernels: no matrix-core figure
    assert bench.mfma_use(c, 1, {"ffn_up": 13.0, "dec_down": 12.0}, "gemma1") is None


def test_profile_lines_parse():
    # the committed rocprofv3 summaries carry the lines bench.py reads
    t = bench.measured_traffic("gemma512", "ffn_up")
    assert t is not None and 1.0e8 < t < 4.0e8
    b = bench.measured_mfma_busy("gemma512", "ffn_up")
    assert b is not None and 0.0 < b < 1.0
    assert bench.measured_traffic("nosuchleg", "ffn_up") is None
    assert bench.measured_mfma_busy("gemma1", "ffn_up") is None
