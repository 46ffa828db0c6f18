"""The oracle's fp16 conversions, activation quantizers, block decoders and load-time requantizer
against the reference's own scalar functions, bit for bit.

tests/golden/ref_scalar.npz holds seeded inputs and the outputs of f32_to_f16, f16_to_f32, f16f,
quantize_q8_0_native, pack_A_i8, pack_A_q3k and gguf_dequant_into as compiled from the
reference's qwen_moe_q3k.c (oracle/ref_scalar.py; the fixture script is
tests/golden/make_ref_scalar.py).  Where the reference build itself is present
(oracle/_ref/libref_scalar.so), fresh inputs are checked against it as well.

The fixture also holds the same functions compiled with a*b - c contracted into FMAs (as the
reference's riscv64 gcc -O3 build may compile them): the decoders' products d*sc*q are exact in
fp32 (an fp16 scale times a 6-bit scale times a 5-bit code fits in 24 bits), so both builds give
the same bits, and the test asserts that too.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as ol

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIX = os.path.join(ROOT, "tests", "golden", "ref_scalar.npz")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_scalar.so")


@pytest.fixture(scope="module")
def z():
    return np.load(FIX)


def orc():
    o = ol.oracle()
    o.orc_f32_to_f16.argtypes = [ctypes.c_float]
    o.orc_f32_to_f16.restype = ctypes.c_uint16
    o.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    o.orc_f16_to_f32.restype = ctypes.c_float
    return o


def oracle_f32_to_f16(x):
    o = orc()
    return np.array([o.orc_f32_to_f16(float(v)) for v in x], np.uint16)


def oracle_f16_to_f32_bits(h):
    o = orc()
    return np.array([o.orc_f16_to_f32(int(v)) for v in h], np.float32).view(np.uint32)


def q8k_as_pack_a_q3k(blocks):
    """The oracle's Q8_K records {f32 d; i8 qs[256]; i16 bsums[16]} in pack_A_q3k's byte layout
    {f32 scale; i16 -sum[16]; i8 qs[256]} (qwen_moe_q3k.c:613-623)."""
    n = blocks.size
    out = np.zeros((n, 292), np.uint8)
    out[:, 0:4] = blocks["d"].astype("<f4").view(np.uint8).reshape(n, 4)
    out[:, 4:36] = (-blocks["bsums"].astype(np.int32)).astype("<i2").view(np.uint8).reshape(n, 32)
    out[:, 36:292] = blocks["qs"].view(np.uint8)
    return out.reshape(-1)


def test_f32_to_f16_truncates_like_the_reference(z):
    x = z["f32_to_f16_in"]
    assert np.array_equal(oracle_f32_to_f16(x), z["f32_to_f16_out"])


def test_f16_to_f32_every_half(z):
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_f16_to_f32_bits(allh)
    # The oracle's float return passes through a Python float (a double), which sets the quiet bit
    # of a signalling NaN; NaN halves are therefore compared with that bit (1 << 22) masked.
    nan = np.isnan(allh.view(np.float16))
    ref = z["f16_to_f32_out"]
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.array_equal(got[nan] | (1 << 22), ref[nan] | (1 << 22))
    # the loader's f16f gives the same bits, and both equal the exact conversion off NaN
    assert np.array_equal(z["f16f_out"], z["f16_to_f32_out"])
    fin = ~np.isnan(allh.view(np.float16))
    assert np.array_equal(got[fin], allh.view(np.float16).astype(np.float32).view(np.uint32)[fin])


def test_quantize_q8_0_native(z):
    x = z["act32_in"]
    got = ol.quantize_q8_0(x)
    assert np.array_equal(got.view(np.uint8).reshape(-1), z["q8_0_out"])


def test_pack_a_i8(z):
    x = z["act32_in"]
    got = ol.quantize_i8(x)
    assert np.array_equal(got.view(np.uint8).reshape(-1), z["pack_a_i8_out"])


def test_pack_a_q3k_is_the_oracles_q8_k(z):
    x = z["act256_in"]
    got = q8k_as_pack_a_q3k(ol.quantize_q8_K(x))
    assert np.array_equal(got, z["pack_a_q3k_out"])


@pytest.mark.parametrize("qt", [ol.Q4_0, ol.Q8_0, ol.Q3_K, ol.Q5_K, ol.Q6_K])
def test_block_decoders(z, qt):
    w = z["dequant%d_in" % qt]
    ref = z["dequant%d_out" % qt]
    got = ol.dequant_row(qt, w, ref.size).view(np.uint32)
    assert np.array_equal(got, ref)
    assert np.array_equal(z["dequant%d_fma_out" % qt], ref)


@pytest.mark.parametrize("qt", [ol.Q8_0, ol.Q5_K, ol.Q6_K])
def test_load_time_requant_to_q8_0(z, qt):
    w = z["requant%d_in" % qt]
    N, K = 16, 4096
    got = ol.requant_q8_0(qt, w.reshape(N, -1).view(np.uint8).view(
        {ol.Q8_0: ol.DT_Q8_0, ol.Q5_K: np.dtype((np.void, 176)), ol.Q6_K: np.dtype((np.void, 210))}[qt]))
    assert np.array_equal(got.view(np.uint8).reshape(-1), z["requant%d_out" % qt])
    assert np.array_equal(z["requant%d_fma_out" % qt], z["requant%d_out" % qt])


@pytest.mark.skipif(not os.path.exists(REF_LIB), reason="reference scalar build (oracle/_ref) not present")
@pytest.mark.parametrize("seed", [11, 12])
def test_fresh_inputs_against_the_reference_build(seed):
    L = ctypes.CDLL(REF_LIB)
    p, sz = ctypes.c_void_p, ctypes.c_size_t
    for name in ("ref_f32_to_f16", "ref_q8_0", "ref_pack_a_i8", "ref_pack_a_q3k"):
        getattr(L, name).argtypes = [p, sz, p]
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(256 * 64) * 10.0 ** rng.uniform(-6, 2)).astype(np.float32)
    h = np.empty(x.size, np.uint16)
    L.ref_f32_to_f16(x.ctypes.data, x.size, h.ctypes.data)
    assert np.array_equal(oracle_f32_to_f16(x[:4096]), h[:4096])
    q = np.empty(x.size // 32 * 34, np.uint8)
    L.ref_q8_0(x.ctypes.data, x.size // 32, q.ctypes.data)
    assert np.array_equal(ol.quantize_q8_0(x).view(np.uint8).reshape(-1), q)
    r = np.empty(x.size // 32 * 38, np.uint8)
    L.ref_pack_a_i8(x.ctypes.data, x.size // 32, r.ctypes.data)
    assert np.array_equal(ol.quantize_i8(x).view(np.uint8).reshape(-1), r)
    r = np.empty(x.size // 256 * 292, np.uint8)
    L.ref_pack_a_q3k(x.ctypes.data, x.size // 256, r.ctypes.data)
    assert np.array_equal(q8k_as_pack_a_q3k(ol.quantize_q8_K(x)), r)
