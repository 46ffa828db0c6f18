"""Pins the CPU oracle (oracle/x100_oracle.c) before the parity tests trust it.

Each oracle function is checked against something other than itself:
  gemm_ref_i8         numpy int64 matmul (closed form), the reference's own gemm_ref_i8 built from
                      its sources (oracle/_ref), golden vectors from that build, invariants.
  fp16 conversions    f16->f32: numpy.float16, exhaustive; f32->f16: the reference's truncation,
                      against a round-toward-zero restatement and hand-computed cases.
  Q8_0 / Q8_K         independent numpy restatements + hand-worked tie cases (rint vs roundf).
  Q4_0 / Q4_K / Q3_K  hand-built blocks with known values; numpy encoders written from the block
  dequant             layout (not from the C decoder); random blocks vs numpy decoders.
  qgemv               float64 dequantize-then-dot of the same quantized operands (closed form);
                      zero-scale / offset special cases; exact linearity in d.
  moe_layer           float64 restatement from dequantized weights, tie-breaking, expert
                      permutation invariance, M rows == M single-row calls, dense n_act = n_exp.
"""
import os

import numpy as np
import pytest

import oracle_lib as ol
import refseq
import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------------------------------------
# int8 GEMM
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (16, 16, 16), (37, 29, 53), (64, 1, 300),
                                   (1, 200, 96), (128, 96, 64)])
def test_gemm_ref_closed_form(M, N, K):
    A, B = synth.gemm_inputs(M, N, K, seed=M * 1000 + N * 10 + K)
    C0 = synth.rand_int8(99, (M, N)).astype(np.int32)
    C = C0.copy()
    ol.gemm_ref_i8(A, B, C)
    expect = C0.astype(np.int64) + A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(C, expect.astype(np.int32))


def test_gemm_ref_golden_from_reference_build():
    """Vectors whose outputs the reference's own gemm_ref_i8 produced (tests/golden/make_golden.py)."""
    g = np.load(os.path.join(GOLDEN, "gemm_ref_i8.npz"))
    n = len([k for k in g.files if k.startswith("A")])
    assert n >= 9
    for i in range(n):
        A, B, C0, C = g["A%d" % i], g["B%d" % i], g["C0_%d" % i], g["C%d" % i]
        out = C0.copy()
        ol.gemm_ref_i8(A, B, out)
        assert np.array_equal(out, C), "golden case %d" % i


def test_gemm_ref_matches_reference_library():
    ref = ol.reference()
    if ref is None:
        pytest.skip("reference not built here (oracle/_ref needs /root/reference)")
    A, B = synth.gemm_inputs(70, 90, 110, seed=5)
    C1 = np.zeros((70, 90), np.int32)
    C2 = np.zeros((70, 90), np.int32)
    ol.gemm_ref_i8(A, B, C1)
    ref.gemm_ref_i8(70, 90, 110, A.ctypes.data, B.ctypes.data, C2.ctypes.data)
    assert np.array_equal(C1, C2)


def test_gemm_ref_invariants():
    A, B = synth.gemm_inputs(40, 24, 64, seed=3)
    C = np.zeros((40, 24), np.int32)
    ol.gemm_ref_i8(A, B, C)
    once = C.copy()
    ol.gemm_ref_i8(A, B, C)                      # accumulate: twice == 2 * product
    assert np.array_equal(C, 2 * once)
    # identity: A . I == A
    I = np.eye(64, dtype=np.int8)
    C = np.zeros((40, 64), np.int32)
    ol.gemm_ref_i8(A, I, C)
    assert np.array_equal(C, A.astype(np.int32))
    # extremes: all -128 -> 16384*K per element
    K = 300
    C = np.zeros((3, 5), np.int32)
    ol.gemm_ref_i8(np.full((3, K), -128, np.int8), np.full((K, 5), -128, np.int8), C)
    assert np.all(C == 16384 * K)
    # threaded variant is the same arithmetic
    A, B = synth.gemm_inputs(96, 80, 200, seed=4)
    C1 = np.zeros((96, 80), np.int32)
    C2 = np.zeros((96, 80), np.int32)
    ol.gemm_ref_i8(A, B, C1)
    ol.gemm_ref_i8(A, B, C2, threads=4)
    assert np.array_equal(C1, C2)


# ------------------------------------------------------------------------------------------------
# fp16
# ------------------------------------------------------------------------------------------------
def test_f16_to_f32_exhaustive():
    o = ol.oracle()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([o.orc_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


np_f16_trunc = refseq.f16_trunc   # round-toward-zero restated from its definition


def test_f32_to_f16_truncates_like_reference():
    """orc_f32_to_f16 is the reference's truncating f32_to_f16 (qwen_moe_hp.c:71-79)."""
    o = ol.oracle()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    # every discarded-bit pattern of the top 3 dropped bits in one binade, the subnormal range
    # and the edges of the fp16 range
    binade = (np.arange(0x3f800000, 0x3f800000 + (1 << 23), 0x400, dtype=np.uint64)).astype(np.uint32)
    sub = np.arange(0x32800000, 0x38900000, 0x800, dtype=np.uint32)
    edges = np.array([0x477fe000, 0x477fefff, 0x477ff000, 0x477fffff, 0x47800000, 0x7f7fffff,
                      0x7f800000, 0xff800000, 0x7fc00000, 0xffc00001], dtype=np.uint32)
    f = np.concatenate([bits, binade, sub, edges]).view(np.float32)
    ref = np_f16_trunc(f)
    got = np.array([o.orc_f32_to_f16(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_hand_computed_truncation_cases():
    """Values worked out by hand from the fp16 format (ulp 2^-10 at 1.0, subnormal step 2^-24)."""
    o = ol.oracle()
    cases = [
        (1.0, 0x3C00),
        (1.0 + 0.75 * 2.0**-10, 0x3C00),      # dropped part 0.75 ulp: truncated, RNE gives 0x3C01
        (1.0 + 1.5 * 2.0**-10, 0x3C01),       # tie: RNE goes to the even 0x3C02
        (-(1.0 + 0.999 * 2.0**-10), 0xBC00),  # sign kept, magnitude truncated
        (127.0 / 127.0 * 0.0234375, 0x2600),  # 3 * 2^-7 exactly representable
        (3.75 * 2.0**-24, 0x0003),            # subnormal d: 3 steps (RNE gives 4)
        (2.0**-24, 0x0001),
        (0.999 * 2.0**-24, 0x0000),           # below the smallest subnormal
        (1e-6 / 127.0, 0x0000),               # the Q8_0 amax floor of 1e-6: d rounds to zero
        (2.0**-14 * (1 - 2.0**-23), 0x03FF),  # just below the normal range: all subnormal bits
        (65535.0, 0x7BFF),                    # 65504, the largest finite fp16
        (65536.0, 0x7C00),                    # exponent past the fp16 range
        (-0.0, 0x8000),
        (float("nan"), 0x7C00),
    ]
    for v, want in cases:
        assert o.orc_f32_to_f16(v) == want, (v, hex(o.orc_f32_to_f16(v)), hex(want))


# ------------------------------------------------------------------------------------------------
# activation quantizers
# ------------------------------------------------------------------------------------------------
def np_q8_0(x):
    b = x.reshape(-1, 32).astype(np.float32)
    amax = np.maximum(np.abs(b).max(axis=1), np.float32(1e-6)).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0)).astype(np.float32)
    q = np.clip(np.rint(b * inv[:, None]), -128, 127).astype(np.int8)
    return np_f16_trunc(d), q


def np_q8_K(x):
    b = x.reshape(-1, 256).astype(np.float32)
    amax = np.abs(b).max(axis=1).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        rep = np.where(d != 0, np.float32(1.0) / d, np.float32(0)).astype(np.float32)
    v = (b * rep[:, None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -128, 127).astype(np.int8)  # half away
    bs = q.reshape(-1, 16, 16).astype(np.int32).sum(axis=2).astype(np.int16)
    return d, q, bs


def test_q8_0_matches_numpy_restatement():
    x = np.concatenate([synth.normal_f32(7, (4096,)), synth.normal_f32(8, (256,)) * 1e-3,
                        np.zeros(64, np.float32)])
    blocks = ol.quantize_q8_0(x)
    d, q = np_q8_0(x)
    assert np.array_equal(blocks["d"], d)
    assert np.array_equal(blocks["qs"], q)


def test_q8_0_ties_round_half_even():
    # amax = 127 -> d = 1, inv = 1: x*inv lands exactly on .5 -> rint rounds to even
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    b = ol.quantize_q8_0(x)
    assert list(b["qs"][0][:7]) == [127, 2, 4, -2, -4, 0, 0]
    assert b["d"][0] == np.float16(1.0).view(np.uint16)


def test_q8_K_matches_numpy_restatement():
    x = np.concatenate([synth.normal_f32(9, (2048,)), np.zeros(256, np.float32),
                        synth.normal_f32(10, (256,)) * 1e-4])
    blocks = ol.quantize_q8_K(x)
    d, q, bs = np_q8_K(x)
    assert np.array_equal(blocks["d"].view(np.uint32), d.view(np.uint32))
    assert np.array_equal(blocks["qs"], q)
    assert np.array_equal(blocks["bsums"], bs)
    assert blocks["d"][8] == 0 and not blocks["qs"][8].any()   # all-zero block


def test_q8_K_ties_round_half_away():
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    b = ol.quantize_q8_K(x)
    assert list(b["qs"][0][:7]) == [127, 3, 4, -3, -4, 1, -1]
    assert b["bsums"][0][0] == 127 + 3 + 4 - 3 - 4 + 1 - 1


# ------------------------------------------------------------------------------------------------
# block dequantization
# ------------------------------------------------------------------------------------------------
F16_ONE = int(np.float16(1.0).view(np.uint16))
F16_HALF = int(np.float16(0.5).view(np.uint16))


def test_q4_0_known_block():
    # qs[j] = j | (15-j)<<4, d = 1: elements j<16 -> j-8 (low nibbles), j>=16 -> (15-(j-16))-8
    blk = np.zeros(1, synth.DT_Q4_0)
    blk["d"] = F16_ONE
    blk["qs"][0] = [j | ((15 - j) << 4) for j in range(16)]
    got = ol.dequant_row(ol.Q4_0, blk, 32)
    expect = [j - 8 for j in range(16)] + [(15 - j) - 8 for j in range(16)]
    assert got.tolist() == [float(v) for v in expect]


def np_q4_K_encode_scales(sc, m):
    """6-bit (sc, m) pairs of the 8 sub-blocks -> 12 bytes, written from the Q4_K layout:
    bytes 0-3 / 4-7 hold sc0-3 / m0-3 in bits 0-5; bytes 8-11 hold the low nibbles of sc4-7
    (bits 0-3) and m4-7 (bits 4-7); the top 2 bits of sc4-7 / m4-7 sit in bits 6-7 of bytes
    0-3 / 4-7."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def test_q4_K_known_block():
    rng = np.random.default_rng(3)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    blk = np.zeros(1, synth.DT_Q4_K)
    blk["d"] = F16_ONE
    blk["dmin"] = F16_HALF
    blk["scales"][0] = np_q4_K_encode_scales(sc, m)
    q = rng.integers(0, 16, 256)   # element value nibble per (sub-block j, l)
    qs = np.zeros(128, np.uint8)
    for j in range(8):
        for l in range(32):
            byte = 32 * (j // 2) + l
            qs[byte] |= (q[32 * j + l] << (4 if j % 2 else 0))
    blk["qs"][0] = qs
    got = ol.dequant_row(ol.Q4_K, blk, 256)
    expect = np.array([1.0 * sc[e // 32] * q[e] - 0.5 * m[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(got, expect)


def np_q3_K_encode_scales(s6):
    """16 six-bit scales -> 12 bytes (Q3_K layout): low nibble of scale i (i<8) in bits 0-3 of
    byte i, of scale i+8 in bits 4-7 of byte i; the top 2 bits of scale i in byte 8+(i%4),
    bits 2*(i//4)."""
    s = np.zeros(12, np.uint8)
    for i in range(16):
        lo, hi = s6[i] & 15, s6[i] >> 4
        s[i % 8] |= lo << (4 * (i // 8))
        s[8 + i % 4] |= hi << (2 * (i // 4))
    return s


def test_q3_K_known_block():
    rng = np.random.default_rng(4)
    s6 = rng.integers(0, 64, 16)
    v = rng.integers(-4, 4, 256)       # element values in [-4, 3]
    hmask = np.zeros(32, np.uint8)
    qs = np.zeros(64, np.uint8)
    for e in range(256):
        h, j, l = e // 128, (e // 32) % 4, e % 32
        low, hbit = (v[e] + 4) & 3, 1 if v[e] >= 0 else 0   # v = low - (hbit ? 0 : 4)
        qs[32 * h + l] |= low << (2 * j)
        hmask[l] |= hbit << (4 * h + j)
    blk = np.zeros(1, synth.DT_Q3_K)
    blk["hmask"][0], blk["qs"][0], blk["scales"][0], blk["d"] = hmask, qs, np_q3_K_encode_scales(s6), F16_ONE
    got = ol.dequant_row(ol.Q3_K, blk, 256)
    sub = [8 * (e // 128) + 2 * ((e // 32) % 4) + (e % 32) // 16 for e in range(256)]
    expect = np.array([(s6[sub[e]] - 32) * v[e] for e in range(256)], np.float32)
    assert np.array_equal(got, expect)


def np_q6_K_encode(q):
    """256 values q in [-32, 31] -> (ql[128], qh[64]) written from the Q6_K layout: in half h
    (elements 128h + p, p < 128) the low 4 bits of q + 32 go to ql[64h + p % 64] (low nibble for
    p < 64, high nibble otherwise) and its top 2 bits to qh[32h + p % 32] at bit 2 * (p // 32)."""
    u = np.asarray(q) + 32
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        h, p = e // 128, e % 128
        ql[64 * h + p % 64] |= (u[e] & 15) << (4 * (p // 64))
        qh[32 * h + p % 32] |= (u[e] >> 4) << (2 * (p // 32))
    return ql, qh


def test_q6_K_known_block():
    rng = np.random.default_rng(5)
    q = rng.integers(-32, 32, 256)
    sc = rng.integers(-128, 128, 16)
    blk = np.zeros(1, synth.DT_Q6_K)
    blk["ql"][0], blk["qh"][0] = np_q6_K_encode(q)
    blk["scales"][0] = sc
    blk["d"] = F16_HALF
    got = ol.dequant_row(ol.Q6_K, blk, 256)
    expect = np.array([0.5 * sc[e // 16] * q[e] for e in range(256)], np.float32)   # 16-element sub-blocks
    assert np.array_equal(got, expect)


def np_q5_K_encode(q):
    """256 values q in [0, 31] -> (qh[32], qs[128]) written from the Q5_K layout: element
    e = 64c + 32hi + l keeps its low 4 bits in qs[32c + l] (low nibble hi = 0, high nibble hi = 1)
    and its fifth bit in qh[l] at bit e // 32."""
    q = np.asarray(q)
    qh = np.zeros(32, np.uint8)
    qs = np.zeros(128, np.uint8)
    for e in range(256):
        c, hi, l = e // 64, (e // 32) % 2, e % 32
        qs[32 * c + l] |= (q[e] & 15) << (4 * hi)
        qh[l] |= (q[e] >> 4) << (e // 32)
    return qh, qs


def test_q5_K_known_block():
    rng = np.random.default_rng(6)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    q = rng.integers(0, 32, 256)
    blk = np.zeros(1, synth.DT_Q5_K)
    blk["d"] = F16_ONE
    blk["dmin"] = F16_HALF
    blk["scales"][0] = np_q4_K_encode_scales(sc, m)   # same 6-bit packing as Q4_K
    blk["qh"][0], blk["qs"][0] = np_q5_K_encode(q)
    got = ol.dequant_row(ol.Q5_K, blk, 256)
    expect = np.array([1.0 * sc[e // 32] * q[e] - 0.5 * m[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(got, expect)


def np_k_scale_min(s):
    """6-bit (sc, m) of the 8 sub-blocks from the 12 scale bytes (Q4_K / Q5_K packing)."""
    s = s.astype(np.int64)
    sh = s.shape[:-1] + (8,)
    sc, mn = np.zeros(sh, np.int64), np.zeros(sh, np.int64)
    sc[..., :4], mn[..., :4] = s[..., 0:4] & 63, s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn


def np_dequant(qtype, W):
    """Vectorised numpy decoders of the three layouts (float64)."""
    N, nb = W.shape
    if qtype == synth.Q4_0:
        d = W["d"].view(np.float16).astype(np.float64)
        lo, hi = (W["qs"] & 15).astype(np.int64) - 8, (W["qs"] >> 4).astype(np.int64) - 8
        return (np.concatenate([lo, hi], axis=2) * d[..., None]).reshape(N, nb * 32)
    if qtype == synth.Q4_K:
        d = W["d"].view(np.float16).astype(np.float64)
        dmin = W["dmin"].view(np.float16).astype(np.float64)
        s = W["scales"].astype(np.int64)
        sc = np.zeros((N, nb, 8), np.int64)
        mn = np.zeros((N, nb, 8), np.int64)
        sc[..., :4], mn[..., :4] = s[..., 0:4] & 63, s[..., 4:8] & 63
        sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
        mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
        qs = W["qs"].reshape(N, nb, 4, 32).astype(np.int64)
        q = np.stack([qs & 15, qs >> 4], axis=3).reshape(N, nb, 8, 32)   # sub-block 2p, 2p+1
        val = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * mn[..., None]
        return val.reshape(N, nb * 256)
    if qtype == synth.Q3_K:
        d = W["d"].view(np.float16).astype(np.float64)
        s = W["scales"].astype(np.int64)
        i = np.arange(16)
        s6 = ((s[..., i % 8] >> (4 * (i // 8))) & 15) | (((s[..., 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)
        e = np.arange(256)
        h, j, l = e // 128, (e // 32) % 4, e % 32
        low = (W["qs"][..., 32 * h + l].astype(np.int64) >> (2 * j)) & 3
        hb = (W["hmask"][..., l].astype(np.int64) >> (4 * h + j)) & 1
        q = low - 4 * (1 - hb)
        sub = 8 * h + 2 * j + l // 16
        return (d[..., None] * (s6[..., sub] - 32) * q).reshape(N, nb * 256)
    if qtype == synth.Q8_0:
        d = W["d"].view(np.float16).astype(np.float64)
        return (W["qs"].astype(np.float64) * d[..., None]).reshape(N, nb * 32)
    e = np.arange(256)
    if qtype == synth.Q5_K:
        d = W["d"].view(np.float16).astype(np.float64)
        dmin = W["dmin"].view(np.float16).astype(np.float64)
        sc, mn = np_k_scale_min(W["scales"])
        c, hi, l = e // 64, (e // 32) % 2, e % 32
        nib = (W["qs"][..., 32 * c + l].astype(np.int64) >> (4 * hi)) & 15
        hb = (W["qh"][..., l].astype(np.int64) >> (e // 32)) & 1
        sub = e // 32
        val = d[..., None] * sc[..., sub] * (nib + 16 * hb) - dmin[..., None] * mn[..., sub]
        return val.reshape(N, nb * 256)
    if qtype == synth.Q6_K:
        d = W["d"].view(np.float16).astype(np.float64)
        h, p = e // 128, e % 128
        low = (W["ql"][..., 64 * h + p % 64].astype(np.int64) >> (4 * (p // 64))) & 15
        top = (W["qh"][..., 32 * h + p % 32].astype(np.int64) >> (2 * (p // 32))) & 3
        q = (low | (top << 4)) - 32
        return (d[..., None] * W["scales"][..., e // 16].astype(np.int64) * q).reshape(N, nb * 256)
    raise ValueError(qtype)


@pytest.mark.parametrize("qtype,K", [(synth.Q4_0, 512), (synth.Q4_K, 1024), (synth.Q3_K, 1024),
                                     (synth.Q8_0, 512), (synth.Q5_K, 1024), (synth.Q6_K, 1024)])
def test_dequant_random_blocks_vs_numpy(qtype, K):
    W = synth.quant_weight(qtype, 6, K, seed=21)
    ref = np_dequant(qtype, W)
    for n in range(6):
        got = ol.dequant_row(qtype, W[n], K)
        np.testing.assert_allclose(got, ref[n], rtol=2e-7, atol=1e-12)


# ------------------------------------------------------------------------------------------------
# quantized GEMV
# ------------------------------------------------------------------------------------------------
I8_PATH = (synth.Q8_0, synth.Q5_K, synth.Q6_K)


def w_dequant(qtype, W):
    """float64 values of the weight the GEMV multiplies (after the load-time requantization
    of the int8 path)."""
    if qtype in I8_PATH:
        return np_dequant(synth.Q8_0, ol.requant_q8_0(qtype, W))
    return np_dequant(qtype, W)


def q8_dequant(qtype, x):
    """Quantize x rows with the oracle, return the float64 values actually multiplied."""
    rows = []
    for r in x:
        if qtype in I8_PATH:
            b = ol.quantize_i8(r)
            rows.append((b["qs"].astype(np.float64) * b["s"].astype(np.float64)[:, None]).ravel())
        elif qtype == synth.Q4_0:
            b = ol.quantize_q8_0(r)
            rows.append((b["qs"].astype(np.float64) * b["d"].view(np.float16).astype(np.float64)[:, None]).ravel())
        else:
            b = ol.quantize_q8_K(r)
            rows.append((b["qs"].astype(np.float64) * b["d"].astype(np.float64)[:, None]).ravel())
    return np.array(rows)


@pytest.mark.parametrize("qtype,N,K,M", [(synth.Q4_0, 64, 1024, 1), (synth.Q4_0, 33, 256, 3),
                                         (synth.Q4_K, 48, 2048, 1), (synth.Q4_K, 20, 768, 4),
                                         (synth.Q3_K, 48, 2048, 1), (synth.Q3_K, 17, 512, 4),
                                         (synth.Q8_0, 40, 1024, 1), (synth.Q8_0, 9, 96, 3),
                                         (synth.Q5_K, 24, 1024, 2), (synth.Q6_K, 30, 2048, 1),
                                         (synth.Q6_K, 11, 512, 4)])
def test_qgemv_closed_form(qtype, N, K, M):
    W = synth.quant_weight(qtype, N, K, seed=N + K)
    x = synth.normal_f32(M * 7 + K, (M, K))
    y = ol.qgemv(qtype, W, x)
    ref = q8_dequant(qtype, x) @ w_dequant(qtype, W).T
    err = np.abs(y - ref)
    assert np.all(err <= 1e-5 * np.abs(ref) + 1e-4 * np.abs(ref).max() * 1e-3 + 1e-6), err.max()


def test_qgemv_special_cases():
    x = synth.normal_f32(1, (2, 512))
    # Q4_0 with every nibble 8 -> all elements 0 -> y == 0 exactly
    W = synth.quant_weight(synth.Q4_0, 5, 512, seed=2)
    W["qs"] = 0x88
    assert not ol.qgemv(synth.Q4_0, W, x).any()
    # Q4_K with all scales / mins 0 -> y == 0
    W = synth.quant_weight(synth.Q4_K, 5, 512, seed=3)
    W["scales"] = 0
    assert not ol.qgemv(synth.Q4_K, W, x).any()
    # Q3_K with every 6-bit scale 32 -> (s - 32) == 0 -> y == 0
    W = synth.quant_weight(synth.Q3_K, 5, 512, seed=4)
    W["scales"] = np_q3_K_encode_scales(np.full(16, 32))
    assert not ol.qgemv(synth.Q3_K, W, x).any()
    # Q4_K dmin-only: sc = 0, m = 1 -> y = -dmin * dx * sum(qx)
    W = synth.quant_weight(synth.Q4_K, 3, 256, seed=5)
    W["scales"] = np_q4_K_encode_scales(np.zeros(8, int), np.ones(8, int))
    y = ol.qgemv(synth.Q4_K, W, x[:1, :256])
    xb = ol.quantize_q8_K(x[0, :256])
    expect = -(xb["d"][0] * W["dmin"][:, 0].view(np.float16).astype(np.float32)) * xb["qs"][0].astype(np.int32).sum()
    np.testing.assert_allclose(y[0], expect, rtol=1e-6)


@pytest.mark.parametrize("qtype,K", [(synth.Q8_0, 256), (synth.Q5_K, 512), (synth.Q6_K, 512)])
def test_requant_q8_0_bound_and_idempotence(qtype, K):
    """Load-time requantization to Q8_0: every 32-group's largest element maps to +-127, every
    element is within half a step (plus the fp16 truncation of the step) of the fp32 dequantized
    value, and requantizing the result again changes nothing (the loader's lossless claim for
    well-formed Q8_0 data, qwen_moe_q3k.c:520-524)."""
    N = 5
    W = synth.quant_weight(qtype, N, K, seed=31)
    R = ol.requant_q8_0(qtype, W)
    assert R.shape == (N, K // 32)
    w = np.stack([ol.dequant_row(qtype, W[n], K) for n in range(N)]).reshape(N, K // 32, 32).astype(np.float64)
    amax = np.maximum(np.abs(w).max(axis=2), 1e-6)
    step = amax / 127.0
    d16 = R["d"].view(np.float16).astype(np.float64)
    # the stored step is the fp32 step truncated to fp16: never above it, less than one fp16 ulp
    # (2^-10 relative) below it
    assert np.all(d16 <= step * (1 + 2.0 ** -23))
    assert np.all(d16 > step * (1 - 2.0 ** -10) * (1 - 2.0 ** -23))
    assert np.all(np.abs(R["qs"]).max(axis=2) == 127)
    err = np.abs(R["qs"].astype(np.float64) * d16[..., None] - w)
    assert np.all(err <= 0.5 * step[..., None] * (1 + 1e-6) + 127 * np.abs(d16 - step)[..., None])
    R2 = ol.requant_q8_0(synth.Q8_0, R)
    assert np.array_equal(R2["d"], R["d"]) and np.array_equal(R2["qs"], R["qs"])


def test_requant_q8_0_rescales_narrow_blocks():
    # a Q8_0 block whose largest |q| is 64 (not 127) is re-encoded with d' = 64*d/127
    W = np.zeros((1, 1), synth.DT_Q8_0)
    W["d"] = F16_ONE
    W["qs"][0, 0] = np.arange(-16, 16)
    W["qs"][0, 0, 0] = 64
    R = ol.requant_q8_0(synth.Q8_0, W)
    assert R["d"][0, 0] == np_f16_trunc(np.float32(64.0) / np.float32(127.0))
    assert R["d"][0, 0] == 0x3808   # 64/127 = 2^-1 * 1.0078740: exponent field 14, mantissa 8.06 -> 8
    inv = np.float32(1.0) / np.float32(np.float32(64.0) / np.float32(127.0))
    expect = np.clip(np.rint(W["qs"][0, 0].astype(np.float32) * inv), -128, 127)
    assert np.array_equal(R["qs"][0, 0], expect.astype(np.int8))


def test_quantize_i8_conventions():
    # fp32 scale = max(amax, 1e-6)/127 (not fp16), ties to even, int16 sum of the 32 values
    x = np.zeros(96, np.float32)
    x[:32] = np.linspace(-3, 3, 32, dtype=np.float32)
    x[0] = 127.0                      # scale 1.0 -> q = rint(x)
    x[1:5] = [2.5, 3.5, -2.5, -0.5]   # ties -> 2, 4, -2, -0
    x[32:64] = synth.normal_f32(3, (32,)) * np.float32(1e-3)
    b = ol.quantize_i8(x)
    assert b["s"][0] == np.float32(1.0)
    assert b["qs"][0][:5].tolist() == [127, 2, 4, -2, 0]
    assert np.array_equal(b["qs"][0].astype(np.float32), np.clip(np.rint(x[:32]), -128, 127))
    amax = np.float32(np.abs(x[32:64]).max())
    assert b["s"][1] == amax / np.float32(127.0) and np.abs(b["qs"][1]).max() == 127
    assert b["s"][2] == np.float32(1e-6) / np.float32(127.0) and not b["qs"][2].any()
    assert all(int(b["asum"][i]) == int(b["qs"][i].astype(np.int32).sum()) for i in range(3))


def test_qgemv_q8w_is_the_per_call_part():
    # the requantize-at-load + per-call split gives exactly the one-call result
    W = synth.quant_weight(synth.Q6_K, 12, 512, seed=14)
    x = synth.normal_f32(15, (3, 512))
    y1 = ol.qgemv(synth.Q6_K, W, x)
    y2 = ol.qgemv_q8w(ol.requant_q8_0(synth.Q6_K, W), x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_qgemv_i8_path_special_cases():
    x = synth.normal_f32(11, (2, 512))
    # Q6_K with every scale 0 -> weights 0 -> requantized d rounds to fp16 0 -> y == 0
    W = synth.quant_weight(synth.Q6_K, 4, 512, seed=7)
    W["scales"] = 0
    assert not ol.qgemv(synth.Q6_K, W, x).any()
    # Q5_K with sc = 0 and m = 1 -> every element -dmin -> y = -dmin * sum over the activation
    W = synth.quant_weight(synth.Q5_K, 3, 512, seed=8)
    W["scales"] = np_q4_K_encode_scales(np.zeros(8, int), np.ones(8, int))
    W["dmin"] = F16_HALF
    y = ol.qgemv(synth.Q5_K, W, x)
    xa = np.stack([(lambda b: (b["qs"].astype(np.float64) * b["s"].astype(np.float64)[:, None]).sum())(ol.quantize_i8(r)) for r in x])
    # requantized weight: every element -0.5 -> d' = fp16 truncation of 0.5/127, q = -127
    dq = float(np_f16_trunc(np.float32(0.5) / np.float32(127.0)).view(np.float16)) * -127
    np.testing.assert_allclose(y, np.repeat((dq * xa)[:, None], 3, axis=1), rtol=1e-5)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q4_K, synth.Q3_K, synth.Q8_0, synth.Q6_K])
def test_qgemv_linear_in_scale(qtype):
    K = 512
    W = synth.quant_weight(qtype, 8, K, seed=6)
    W["d"] = np.float16(0.25).view(np.uint16)
    x = synth.normal_f32(2, (1, K))
    y1 = ol.qgemv(qtype, W, x)
    W2 = W.copy()
    W2["d"] = np.float16(0.5).view(np.uint16)
    if qtype == synth.Q4_K:
        W2["dmin"] = (W["dmin"].view(np.float16) * np.float16(2)).view(np.uint16)
    y2 = ol.qgemv(qtype, W2, x)
    assert np.array_equal(y2, 2 * y1)   # powers of two: exact


# ------------------------------------------------------------------------------------------------
# MoE layer
# ------------------------------------------------------------------------------------------------
def small_moe(seed, n_exp=16, d=512, ff=256):
    Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed)
    R = synth.moe_router(n_exp, d, seed + 1)
    return Wg, Wu, Wd, R


def np_moe(hn, R, Wg, Wu, Wd, n_act):
    """float64 restatement of the layer from dequantized weights and the oracle's quantizers."""
    out = np.zeros(hn.shape, np.float64)
    for m, h in enumerate(hn):
        lg = R.astype(np.float64) @ h.astype(np.float64)
        p = np.exp(lg - lg.max())
        p /= p.sum()
        sel = sorted(range(len(p)), key=lambda e: (-p[e], e))[:n_act]
        w = p[sel] / p[sel].sum()
        xq = q8_dequant(synth.Q4_K, h[None])[0]
        for a, e in enumerate(sel):
            g = np_dequant(synth.Q4_K, Wg[e]) @ xq
            u = np_dequant(synth.Q4_K, Wu[e]) @ xq
            act = (g / (1 + np.exp(-g)) * u).astype(np.float32)
            aq = q8_dequant(synth.Q4_K, act[None])[0]
            out[m] += w[a] * (np_dequant(synth.Q4_K, Wd[e]) @ aq)
    return out


def test_moe_matches_float64_restatement():
    Wg, Wu, Wd, R = small_moe(30)
    hn = synth.normal_f32(31, (2, 512))
    out, sel, sw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act=4)
    ref = np_moe(hn, R, Wg, Wu, Wd, 4)
    # activation re-quantization may flip a rounding at a .5 boundary; compare at 1e-3 of scale
    assert np.abs(out - ref).max() <= 2e-3 * np.abs(ref).max()
    np.testing.assert_allclose(sw.sum(axis=1), 1.0, rtol=1e-6)


def test_moe_router_ties_lower_index_wins():
    n_exp, d = 8, 256
    R = np.zeros((n_exp, d), np.float32)
    R[[2, 5, 6]] = 1.0           # three equal top logits
    hn = np.ones((1, d), np.float32)
    _, sel, sw = ol.moe_route(hn, R, 4)
    assert sel[0].tolist()[:3] == [2, 5, 6]
    assert sel[0][3] == 0         # remaining experts tie at the next value: lowest id first
    assert abs(sw[0][:3].sum() + sw[0][3] - 1) < 1e-6


def test_moe_rows_independent_and_permutation_invariant():
    Wg, Wu, Wd, R = small_moe(40)
    hn = synth.normal_f32(41, (3, 512))
    out, sel, sw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act=4)
    for m in range(3):   # M rows == M single-row calls (per-row activation quantization)
        o1, s1, w1 = ol.moe_layer(hn[m:m + 1], R, Wg, Wu, Wd, n_act=4)
        assert np.array_equal(o1[0], out[m]) and np.array_equal(s1[0], sel[m])
    perm = np.random.default_rng(0).permutation(R.shape[0])
    outp, selp, _ = ol.moe_layer(hn, R[perm], Wg[perm], Wu[perm], Wd[perm], n_act=4)
    assert np.array_equal(perm[selp], sel)
    np.testing.assert_allclose(outp, out, rtol=1e-5, atol=1e-5 * np.abs(out).max())


def test_moe_residual_flag():
    Wg, Wu, Wd, R = small_moe(50)
    hn = synth.normal_f32(51, (1, 512))
    base = synth.normal_f32(52, (1, 512))
    out, _, _ = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act=2)
    res, _, _ = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act=2, out=base.copy(), residual=True)
    assert np.array_equal(res, base + out)


def test_swiglu_is_exact_silu_product():
    o = ol.oracle()
    for g, u in [(0.0, 3.0), (1.5, -2.0), (-30.0, 1.0), (12.0, 0.5), (-0.25, 4.0)]:
        g32, u32 = np.float32(g), np.float32(u)
        e = np.float32(np.exp(-np.float64(g32)))
        expect = np.float32(np.float32(g32 / np.float32(1 + e)) * u32)
        assert np.float32(o.orc_swiglu(g32, u32)) == expect
