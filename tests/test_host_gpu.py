"""The C host programs over libx100hip (x100-gemm_amd/host/, built into x100-gemm_amd/bin/):
  q4_gemv     the reference's bench/q4_gemv.c command line, output lines and exit status;
  x100_host   the integration guide's C code (lin_hip_new / lin_hip_mm, moe_layer_hip and its
              _ws / _noalloc forms) fed the oracle's inputs through files, outputs compared with
              the oracle bit for bit;
  moe_decode  the decode weight stream of bench/moe_decode.c with --check: every launch of the
              stacked-launch stream, and the graph-replayed token, against a host matmul."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as ol
import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "x100-gemm_amd", "bin")


def run(args, timeout=120):
    exe = os.path.join(BIN, args[0])
    assert os.path.exists(exe), "%s not built (make -C x100-gemm_amd)" % exe
    print("run:", " ".join(str(a) for a in args), flush=True)
    return subprocess.run([exe] + [str(a) for a in args[1:]], capture_output=True, text=True, timeout=timeout)


# ---- q4_gemv --------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K,M", [(4864, 896, 1), (4864, 896, 4), (4096, 4096, 8), (8, 32, 1)])
def test_q4_gemv_cli(dev, N, K, M):
    out = run(["q4_gemv", N, K, M, 1, 20])
    assert out.returncode == 0, out.stdout + out.stderr
    assert "int4 GEMV %dx%d M=%d: y==ref OK (0/%d mismatch)" % (N, K, M, N * M) in out.stdout
    assert "int8 GEMV: y==ref OK (0/%d mismatch)" % (N * M) in out.stdout
    assert "ms/GEMV" in out.stdout


def test_q4_gemv_cli_bad_dims(dev):
    for args in ((4864, 900), (100, 896), (4864, 896, 9)):
        out = run(["q4_gemv", *args])
        assert out.returncode == 2, out.stdout
        assert "need N%8,K%32" in out.stdout


def test_q4_gemv_cli_draws_the_reference_inputs(dev):
    """The int4 sample outputs equal a host matmul of the reference's rand() draws (srand(7))."""
    import ctypes
    libc = ctypes.CDLL("libc.so.6")
    N, K, M = 16, 64, 2
    libc.srand(7)
    W = np.array([libc.rand() % 15 - 7 for _ in range(N * K)], np.int64).reshape(N, K)
    x = np.array([libc.rand() % 256 - 128 for _ in range(M * K)], np.int64).reshape(M, K)
    y = x @ W.T
    out = run(["q4_gemv", N, K, M, 1, 3])
    assert out.returncode == 0, out.stdout + out.stderr
    line = [l for l in out.stdout.splitlines() if l.startswith("samples")][0]
    ref = [int(v) for v in line.split("ref:")[1].split("|")[0].split()]
    assert ref == y[0, :4].tolist()


# ---- x100_host: the integration guide's C code ------------------------------------------------
@pytest.mark.parametrize("qtype,N,K,M", [(synth.Q4_0, 4096, 4096, 1), (synth.Q4_K, 6144, 2048, 4),
                                         (synth.Q3_K, 6144, 2048, 1), (synth.Q5_K, 2048, 4096, 1),
                                         (synth.Q6_K, 1000, 2048, 3), (synth.Q8_0, 512, 2048, 8)])
def test_c_lin_hip(dev, tmp_path, qtype, N, K, M):
    W = synth.quant_weight(qtype, N, K, seed=1300 + qtype)
    x = synth.normal_f32(1301 + M, (M, K))
    w_f, x_f, y_f = tmp_path / "w.bin", tmp_path / "x.bin", tmp_path / "y.bin"
    np.ascontiguousarray(W).tofile(w_f)
    x.tofile(x_f)
    out = run(["x100_host", "lin", qtype, N, K, M, w_f, x_f, y_f])
    assert out.returncode == 0, out.stderr
    y = np.fromfile(y_f, np.float32).reshape(M, N)
    ref = ol.qgemv(qtype, W, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M,mode", [(1, ""), (4, ""), (4, "ws"), (8, "noalloc"), (16, "ws")])
def test_c_moe_layer(dev, tmp_path, M, mode):
    n_exp, d, ff, n_act = 128, 2048, 768, 8
    Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed=500)
    R = synth.moe_router(n_exp, d, seed=501)
    hn = synth.normal_f32(1400 + M, (M, d))
    files = {}
    for name, a in (("hn", hn), ("R", R), ("Wg", Wg), ("Wu", Wu), ("Wd", Wd)):
        files[name] = tmp_path / (name + ".bin")
        np.ascontiguousarray(a).tofile(files[name])
    out_f = tmp_path / "out.bin"
    args = ["x100_host", "moe", M, d, ff, n_exp, n_act, files["hn"], files["R"], files["Wg"], files["Wu"],
            files["Wd"], out_f] + ([mode] if mode else [])
    out = run(args)
    assert out.returncode == 0, out.stderr
    raw = np.fromfile(out_f, np.uint8)
    o = raw[:M * d * 4].view(np.float32).reshape(M, d)
    sel = raw[M * d * 4:M * d * 4 + M * n_act * 4].view(np.int32).reshape(M, n_act)
    sw = raw[M * d * 4 + M * n_act * 4:].view(np.float32).reshape(M, n_act)
    ref, rsel, rsw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act)
    assert np.array_equal(sel, rsel)
    assert np.array_equal(sw.view(np.uint32), rsw.view(np.uint32))
    assert np.array_equal(o.view(np.uint32), ref.view(np.uint32))


# ---- moe_decode ------------------------------------------------------------------------------------
def test_moe_decode_stream_check(dev):
    """Two layers of the Qwen3-30B-A3B stream, q4 and q8, M = 1 and an M = 8 verify pass at U = 8
    and 24: every launch and the graph-replayed lm_head equal the host matmul."""
    out = run(["moe_decode", "--layers", 2, "--reps", 2, "--us", "8,24", "--check", "--json"], timeout=300)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    assert "check: every launch equals the host matmul" in out.stdout
    import json
    res = json.loads(out.stdout.strip().splitlines()[-1])
    assert res["check"] is True and res["layers"] == 2
    assert res["q4"]["m1_ms_per_token"] > 0 and res["q8"]["m8_u24_ms_per_pass"] > 0
