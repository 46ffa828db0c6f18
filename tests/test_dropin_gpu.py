"""The reference's own GEMM harness (bench/bench.c), built from its sources with gemm_ime_i8 taken
from libx100hip.so instead of src/gemm_ime_i8.c (oracle/Makefile target `dropin`), runs on the
GPU and reports zero mismatches against its own gemm_ref_i8 (bench/bench.c:79-91)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "gemm_bench_hip")

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not os.path.exists(BIN), reason="oracle/_ref/gemm_bench_hip not built (needs the reference sources)")
@pytest.mark.parametrize("shape", [("256", "256", "256"), ("100", "300", "520"), ("512", "512", "512")])
def test_reference_harness_on_gpu(dev, shape):
    out = subprocess.run([BIN, *shape, "3"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    line = [l for l in out.stdout.splitlines() if "i8->i32" in l]
    assert line, out.stdout
    assert re.search(r"mismatch=0\s+OK", line[0]), line[0]
