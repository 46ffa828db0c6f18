"""Writes tests/golden/ref_scalar.npz: inputs and outputs of the reference's own scalar format
functions, run from oracle/_ref/libref_scalar.so (built by `make -C oracle refscalar`, which
compiles f32_to_f16, f16_to_f32, f16f, quantize_q8_0_native, pack_A_i8, pack_A_q3k and
gguf_dequant_into out of the reference's qwen_moe_q3k.c), and from libref_scalar_fma.so (the same
text compiled with a*b - c fused into FMAs, as the reference's riscv64 gcc -O3 build may).

Only data is written: seeded inputs and the reference functions' outputs.  Run from the repo root:

    make -C oracle refscalar && python tests/golden/make_ref_scalar.py
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "x100-gemm_amd"))
import synth  # noqa: E402

LIB = os.path.join(ROOT, "oracle", "_ref", "libref_scalar.so")
LIB_FMA = os.path.join(ROOT, "oracle", "_ref", "libref_scalar_fma.so")
OUT = os.path.join(ROOT, "tests", "golden", "ref_scalar.npz")


def load(path):
    L = ctypes.CDLL(path)
    p, sz, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32
    for name in ("ref_f32_to_f16", "ref_f16_to_f32", "ref_f16f", "ref_q8_0", "ref_pack_a_i8", "ref_pack_a_q3k"):
        getattr(L, name).argtypes = [p, sz, p]
    L.ref_dequant.argtypes = [u32, p, sz, p]
    L.ref_requant_q8_0.argtypes = [u32, p, sz, sz, sz, p]
    return L


def f32_cases(seed=1):
    """Floats for the fp16 conversions: special values, every binade from 2^-30 to 2^20 (below the
    fp16 subnormals to past the fp16 maximum) with random mantissas, and values just around the
    fp16 rounding points."""
    rng = np.random.default_rng(seed)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 65536.0, 1e6, -1e6,
                        2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26, 5.96e-8, 6.1e-5, 1.0, -1.0,
                        np.float32(1e-45), -np.float32(1e-38)], np.float32)
    e = rng.integers(-30, 21, 20000)
    m = rng.random(20000) + 1.0
    s = np.where(rng.random(20000) < 0.5, -1.0, 1.0)
    binades = (s * m * 2.0 ** e).astype(np.float32)
    # fp16 values plus / minus a fraction of their ulp (truncation vs rounding boundaries)
    h = rng.integers(0, 0x7c00, 5000).astype(np.uint16).view(np.float16).astype(np.float32)
    ulp = np.abs(h) * 2.0 ** -11
    near = np.concatenate([h + ulp * 0.5, h + ulp * 0.49, h - ulp * 0.51, h + ulp * 0.999]).astype(np.float32)
    return np.concatenate([special, binades, near]).astype(np.float32)


def act_cases(seed, n, group):
    """n groups of `group` floats: N(0,1) times a per-group scale from 1e-8 to 1e3, a few all-zero
    groups, groups with one large outlier, and groups on exact half-integer multiples of the scale
    (rounding ties)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, group)).astype(np.float32)
    scale = (10.0 ** rng.uniform(-8, 3, n)).astype(np.float32)
    x *= scale[:, None]
    x[::97] = 0.0
    x[5::61, 3] *= 300.0
    ties = (rng.integers(-254, 255, (n // 16, group)) * 0.5).astype(np.float32)
    ties[:, 0] = 127.0   # amax 127: d = 1, so x * (1/d) lands exactly on the half-integers
    x[7::16][:ties.shape[0]] = ties[:x[7::16].shape[0]]
    return np.ascontiguousarray(x.reshape(-1))


def main():
    L, F = load(LIB), load(LIB_FMA)
    out = {}
    x = f32_cases()
    h = np.empty(x.size, np.uint16)
    L.ref_f32_to_f16(x.ctypes.data, x.size, h.ctypes.data)
    out["f32_to_f16_in"], out["f32_to_f16_out"] = x, h
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for name in ("f16_to_f32", "f16f"):
        y = np.empty(65536, np.float32)
        getattr(L, "ref_" + name)(allh.ctypes.data, 65536, y.ctypes.data)
        out[name + "_out"] = y.view(np.uint32)

    a = act_cases(2, 4096, 32)
    q = np.empty(4096 * 34, np.uint8)
    L.ref_q8_0(a.ctypes.data, 4096, q.ctypes.data)
    r = np.empty(4096 * 38, np.uint8)
    L.ref_pack_a_i8(a.ctypes.data, 4096, r.ctypes.data)
    out["act32_in"], out["q8_0_out"], out["pack_a_i8_out"] = a, q, r
    a = act_cases(3, 1024, 256)
    r = np.empty(1024 * 292, np.uint8)
    L.ref_pack_a_q3k(a.ctypes.data, 1024, r.ctypes.data)
    out["act256_in"], out["pack_a_q3k_out"] = a, r

    for qt in (synth.Q4_0, synth.Q8_0, synth.Q3_K, synth.Q5_K, synth.Q6_K):
        N, K = 8, 2048
        W = np.ascontiguousarray(synth.quant_weight(qt, N, K, seed=300 + qt)).view(np.uint8).reshape(-1)
        for tag, lib in (("", L), ("_fma", F)):
            y = np.empty(N * K, np.float32)
            assert lib.ref_dequant(qt, W.ctypes.data, N * K, y.ctypes.data) == 0
            out["dequant%d%s_out" % (qt, tag)] = y.view(np.uint32)
        out["dequant%d_in" % qt] = W
    for qt in (synth.Q8_0, synth.Q5_K, synth.Q6_K):
        N, K = 16, 4096
        W = np.ascontiguousarray(synth.quant_weight(qt, N, K, seed=400 + qt)).view(np.uint8)
        rb = W.size // N
        for tag, lib in (("", L), ("_fma", F)):
            q = np.empty(N * (K // 32) * 34, np.uint8)
            assert lib.ref_requant_q8_0(qt, W.ctypes.data, N, K, rb, q.ctypes.data) == 0
            out["requant%d%s_out" % (qt, tag)] = q
        out["requant%d_in" % qt] = W.reshape(-1)
    np.savez_compressed(OUT, **out)
    print("wrote %s (%d arrays, %d bytes)" % (OUT, len(out), os.path.getsize(OUT)))


if __name__ == "__main__":
    main()
