"""Host proof of the arithmetic identities behind the division-free activation quantizers
(x100_common.h: div127_rn, f16_trunc_pos, the 1.5 * 2^23 rounding).  The GPU's own v_rcp_f32-based
reciprocal is checked on the device (test_qgemv_gpu.py)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE = os.path.join(HERE, "..", "oracle")


def test_quantizer_identities_hold_for_every_float(tmp_path):
    lib = os.path.join(ORACLE, "liboracle.so")
    if not os.path.exists(lib):
        pytest.skip("oracle not built")
    exe = str(tmp_path / "quant_exact")
    subprocess.check_call(["gcc", "-O2", "-mfma", "-I", ORACLE, os.path.join(HERE, "quant_exact.c"), "-o", exe,
                           "-L", ORACLE, "-loracle", "-Wl,-rpath," + os.path.abspath(ORACLE), "-lm"])
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=300).stdout.split()
    bad_div, bad_f16, bad_round = (int(v) for v in out)
    assert bad_div == 0, "amax / 127 by product + FMA differs for %d inputs" % bad_div
    assert bad_f16 == 0, "fp16 truncation shortcut differs for %d inputs" % bad_f16
    assert bad_round == 0, "1.5 * 2^23 rounding differs from lrintf for %d inputs" % bad_round
