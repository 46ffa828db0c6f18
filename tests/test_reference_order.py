"""The oracle against the reference's own checking arithmetic (tests/refseq.py) at the benchmark
configurations, element-wise rel 1e-3 / abs 1e-4 in fp32.

The oracle takes its sums in the HIP kernels' order (the GPU tests require bit identity with it);
the reference checks its kernels in another order (per-block fp32 sums for Q4_0 and the int8 path,
bench/vendor_ime_a2_full.c:240-259 and bench/vendor_ime_i8_full.c:182-190; double accumulation
of fp32-decoded weights for the K-quants, bench/q3k_probe.c:443-456; the sequential MoE block of
qwen_moe.c:294-311).  These tests bound the distance between the two orders.

Every GEMV configuration meets the tolerance on every element.  The MoE layer meets it except for
elements whose error is explained, and checked here, by one of two causes that no fp32 order can
avoid:
  * conditioning: the output is a small difference of large expert terms (sum_a w_a * y_a with
    |w_a * y_a| up to 1e5 times |out|), so one fp32 rounding of a term already exceeds the
    tolerance; the error must lie within COND_ULPS fp32 ulps of the terms' magnitude;
  * an activation requantization flip: silu(g) * u computed from gate / up values that differ in
    their last bit lands on the other side of a Q8_K rounding boundary, changing one int8 by 1;
    the error must lie within the flip's contribution w_a * d_act * |W[j, k]| (plus the
    conditioning allowance).
The number of such elements is capped at the count measured when these tests were written."""
import numpy as np
import pytest

import oracle_lib as ol
import refseq
import synth

RTOL, ATOL = 1e-3, 1e-4
COND_ULPS = 16           # allowance for fp32 evaluation-order differences, in ulps of the terms


def outside(got, ref):
    return np.abs(got - ref) > ATOL + RTOL * np.abs(ref)


def assert_within(got, ref, what):
    bad = outside(got, ref)
    ratio = float((np.abs(got - ref) / (ATOL + RTOL * np.abs(ref))).max())
    assert not bad.any(), "%s: %d of %d outside rel 1e-3 / abs 1e-4 (worst %.2fx)" % (
        what, int(bad.sum()), bad.size, ratio)
    return ratio


# ------------------------------------------------------------------------------------------------
# GEMVs at the benchmark shapes (the seeds of tests/test_qgemv_gpu.py)
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 4])
def test_q4_0_4096_reference_order(M):
    W = synth.quant_weight(synth.Q4_0, 4096, 4096, 300 + M)
    x = synth.normal_f32(301 + M, (M, 4096))
    r = assert_within(ol.qgemv(synth.Q4_0, W, x), refseq.gemv(synth.Q4_0, W, x), "Q4_0 M=%d" % M)
    print("Q4_0 4096x4096 M=%d: worst element at %.3f of the tolerance" % (M, r))


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q3_K])
@pytest.mark.parametrize("M", [1, 4])
def test_kquant_6144x2048_reference_order(qtype, M):
    W = synth.quant_weight(qtype, 6144, 2048, 400 + M + qtype)
    x = synth.normal_f32(401 + M + qtype, (M, 2048))
    r = assert_within(ol.qgemv(qtype, W, x), refseq.gemv(qtype, W, x), "qtype %d M=%d" % (qtype, M))
    print("qtype %d 6144x2048 M=%d: worst element at %.3f of the tolerance" % (qtype, M, r))


@pytest.mark.parametrize("qtype,N,K", [(synth.Q8_0, 512, 2048),      # attn_k
                                       (synth.Q5_K, 2048, 4096),     # attn_output
                                       (synth.Q6_K, 4096, 2048)])    # lm_head rows
@pytest.mark.parametrize("M", [1, 4])
def test_int8_path_reference_order(qtype, N, K, M):
    W = synth.quant_weight(qtype, N, K, 77 + qtype)
    x = synth.normal_f32(78 + M, (M, K))
    # the load-time requantization is the reference's, bit for bit (truncated fp16 scales)
    R = ol.requant_q8_0(qtype, W)
    d16, q = refseq.requant_q8_0(qtype, W)
    assert np.array_equal(R["d"], d16) and np.array_equal(R["qs"], q)
    assert_within(ol.qgemv(qtype, W, x), refseq.gemv(qtype, W, x), "int8 path qtype %d M=%d" % (qtype, M))


def test_q8_0_activation_scale_is_truncated():
    """Q4_0 parity hinges on the activation scale's fp16 conversion: with the reference's
    truncation the oracle's quantized x is the reference's, byte for byte."""
    x = synth.normal_f32(302, (1, 4096))
    b = ol.quantize_q8_0(x[0])
    d16, _, q = refseq.quant_q8_0(x)
    assert np.array_equal(b["d"], d16[0]) and np.array_equal(b["qs"], q[0])
    # and at this seed many scales differ from round-to-nearest: the convention is exercised
    d32 = (np.maximum(np.abs(x.reshape(-1, 32)).max(axis=1), np.float32(1e-6)) / np.float32(127)).astype(np.float32)
    assert (d32.astype(np.float16).view(np.uint16) != d16[0]).sum() > 20


# ------------------------------------------------------------------------------------------------
# MoE layer, Qwen3-30B-A3B shape (the seeds of tests/test_moe_gpu.py)
# ------------------------------------------------------------------------------------------------
# measured elements outside tolerance per token-row count, each explained by conditioning or a flip
MOE_EXCEPTIONS = {1: 0, 4: 7, 8: 1}

_moe = {}


def moe_case(M, seed=500):
    if "w" not in _moe:
        _moe["w"] = synth.moe_weights(128, 2048, 768, seed) + (synth.moe_router(128, 2048, seed + 1),)
    Wg, Wu, Wd, R = _moe["w"]
    hn = synth.normal_f32(seed + 2 + M, (M, 2048))
    return Wg, Wu, Wd, R, hn


@pytest.mark.parametrize("M", [1, 4, 8])
def test_moe_reference_order(M):
    Wg, Wu, Wd, R, hn = moe_case(M)
    out, sel, sw = ol.moe_layer(hn, R, Wg, Wu, Wd, 8)
    ref, rsel, rsw, probs, acts = refseq.moe_layer(hn, R, Wg, Wu, Wd, 8)

    # routing: same experts, weights within a few ulps, and a top-8 margin far above the
    # difference between the two router orders
    assert np.array_equal(sel, rsel)
    np.testing.assert_allclose(sw, rsw, rtol=1e-5)
    logits, _, _ = ol.moe_route(hn, R, 8)
    srt = -np.sort(-probs, axis=1)
    margin = srt[:, 7] - srt[:, 8]
    lg_ref, _, _, _ = refseq.route(hn, R, 8)
    dlogit = float(np.abs(logits - lg_ref).max())
    print("M=%d: top-8 probability margins %s, router logit difference %.2e" % (M, np.round(margin, 6), dlogit))
    # a logit change dl moves p_i by at most 2 * p_i * max|dl|: the margin is over 100x that
    assert margin.min() > 5e-5 and margin.min() > 100 * 2 * srt[:, 0].max() * dlogit

    # gate / up of every chosen expert: the K-quant GEMV gap, within tolerance
    gu = {}
    for m in range(M):
        for e in sel[m]:
            g_o = ol.qgemv(synth.Q4_K, Wg[e], hn[m:m + 1])[0]
            u_o = ol.qgemv(synth.Q4_K, Wu[e], hn[m:m + 1])[0]
            wg, wu = refseq.dequant_f32(synth.Q4_K, Wg[e]), refseq.dequant_f32(synth.Q4_K, Wu[e])
            assert_within(g_o, refseq.gemv_kquant(synth.Q4_K, None, hn[m:m + 1], wg)[0], "gate m=%d e=%d" % (m, e))
            assert_within(u_o, refseq.gemv_kquant(synth.Q4_K, None, hn[m:m + 1], wu)[0], "up m=%d e=%d" % (m, e))
            gu[(m, int(e))] = (g_o, u_o)

    # the reference's order fed with the oracle's gate / up: the activations are then the
    # oracle's, so only the down projection and the weighted sum differ in order
    ref_o, _, _, _, acts_o = refseq.moe_layer(hn, R, Wg, Wu, Wd, 8, gate_up=lambda m, e: gu[(m, e)])

    # magnitudes: t[m, j] = sum_a w_a * sum_k |W_e(a)[j, k] * act_q[k]|  (the terms' size)
    t = np.zeros((M, 2048))
    flip_bound = np.zeros((M, 2048))
    nflips = 0
    for m in range(M):
        for a in range(8):
            e = int(sel[m, a])
            wd = refseq.dequant_f32(synth.Q4_K, Wd[e]).astype(np.float64)
            d, q = refseq.quant_q8_K(acts_o[m, a][None])
            aq = (q.astype(np.float64) * d.astype(np.float64)[..., None]).ravel()
            t[m] += float(sw[m, a]) * (np.abs(wd) @ np.abs(aq))
            d_r, q_r = refseq.quant_q8_K(acts[m, a][None])
            fl = np.flatnonzero(q_r.ravel() != q.ravel())
            nflips += len(fl)
            for k in fl:   # a changed int8 (and its block scale) moves y[j] by about d * |W[j, k]|
                dk = max(float(d.ravel()[k // 256]), float(d_r.ravel()[k // 256]))
                flip_bound[m] += float(sw[m, a]) * dk * np.abs(wd[:, k]) * abs(int(q_r.ravel()[k]) - int(q.ravel()[k]))
    cond = COND_ULPS * 2.0 ** -24 * t
    tol = ATOL + RTOL * np.abs(ref)

    # 1. oracle vs reference order with the same activations: tolerance or conditioning
    err_o = np.abs(out - ref_o)
    assert np.all(err_o <= ATOL + RTOL * np.abs(ref_o) + cond), "unexplained difference in the down projection"
    # 2. oracle vs the reference's order throughout: tolerance, conditioning or a flip
    err = np.abs(out - ref)
    assert np.all(err <= tol + cond + 1.01 * flip_bound), "unexplained difference"
    bad = np.argwhere(err > tol)
    for m, j in bad:
        print("  row %d col %d: oracle %.6g reference order %.6g (%.1fx tolerance); terms %.3g, "
              "flip allowance %.3g" % (m, j, out[m, j], ref[m, j], err[m, j] / tol[m, j], t[m, j], flip_bound[m, j]))
    print("M=%d: %d of %d outside tolerance, %d activation int8 flips" % (M, len(bad), out.size, nflips))
    assert len(bad) <= MOE_EXCEPTIONS[M]
    assert nflips <= 2
