"""The reference's own checking arithmetic for the quantized products, restated in numpy.

Test infrastructure.  The oracle (oracle/x100_oracle.c) and the HIP kernels share one fixed
summation order (lane-strided partial sums and their reductions), bit for bit.  This module
computes the same products in the order the reference itself uses when it checks its kernels, so
the tests can measure how far that shared order is from the reference's at the benchmark
configurations (element-wise rel 1e-3 / abs 1e-4 in fp32):

  fp16 scales      f32_to_f16 of qwen_moe_hp.c:71-79 (truncation), restated from the definition
                   of round-toward-zero rather than from the bit layout (f16_trunc)
  Q8_0 activation  quantize_q8_0_native, qwen_moe_hp.c:408-414
  Q8_K activation  pack_A_q3k, qwen_moe_q3k.c:612-624
  int8 activation  pack_A_i8, qwen_moe_hp.c:420-427 (qwen_moe_q3k.c:420-427)
  Q4_0 x Q8_0      bench/vendor_ime_a2_full.c:240-259: per 32-block an fp32 running sum of
                   ((q_a * s_a) * (q_w - 8)) * d_w in element order, the block sums added to the
                   row in block order
  int8 path        bench/vendor_ime_i8_full.c:182-190: the same per-block fp32 form with signed
                   q_w; weights requantized at load as lin_new_i8 does (qwen_moe_q3k.c:872-886)
  K-quants         bench/q3k_probe.c:443-456: weights dequantized to fp32 by the reference's
                   decoders (dequantize_q3_K_block qwen_moe_q3k.c:557-577; the Q4_K form
                   d1 * q - m1 of repack.cpp:950-970 / qwen_moe_q3k.c:540-551), activation from
                   its own stored int8 and scale, accumulated in double
  MoE layer        qwen_moe.c:294-311: sequential fp32 router dot, softmax with max-subtract,
                   expf and a sequential sum (qwen_moe.c:189), top-k by strict '>' (lower index
                   wins ties), sequential renormalisation, g / (1 + expf(-g)) * u, down
                   projection, eout += w_a * y_a in slot order

expf: the reference calls libm's expf (glibc's is within 0.502 ulp, i.e. correctly rounded except
when the exact value lies within 0.002 ulp of a rounding midpoint); it is stood in for here by
exp evaluated in binary64 and rounded once to binary32.  Products and sums round in fp32 exactly
as written (no fused multiply-add); where the reference's own build may contract an expression,
the two differ by rounding only.
"""
import numpy as np

import synth

F32 = np.float32


# ------------------------------------------------------------------------------------------------
# fp16
# ------------------------------------------------------------------------------------------------
def f16_trunc(f):
    """fp32 -> fp16 bits by round-toward-zero: numpy's round-to-nearest result, moved one fp16
    step toward zero wherever it overshoots |f|; magnitudes of 2^16 and more, infinities and NaN
    give a signed infinity (the exponent-overflow branch of qwen_moe_hp.c:77)."""
    f = np.asarray(f, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        r = np.atleast_1d(f.astype(np.float16))
        over = np.abs(r.astype(np.float32)) > np.abs(np.atleast_1d(f))
    bits = r.view(np.uint16).copy()
    bits[over] -= 1                      # fp16 magnitudes are monotonic in their bits
    sign = (np.atleast_1d(f).view(np.uint32) >> 16).astype(np.uint16) & np.uint16(0x8000)
    big = ~(np.abs(np.atleast_1d(f)) < np.float32(65536.0))   # includes inf and NaN
    bits[big] = sign[big] | np.uint16(0x7C00)
    return bits.reshape(f.shape)


def f16_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------------------------------------------
# activation quantizers (rows of x, float32)
# ------------------------------------------------------------------------------------------------
def quant_q8_0(x):
    """quantize_q8_0_native per row: returns (fp16 bits of d, fp32 d, q[M][K/32][32])."""
    x = np.asarray(x, np.float32)
    b = x.reshape(x.shape[0], -1, 32)
    amax = np.maximum(np.abs(b).max(axis=2), F32(1e-6))
    d = (amax / F32(127.0)).astype(np.float32)
    inv = (F32(1.0) / d).astype(np.float32)
    q = np.clip(np.rint(b * inv[..., None]), -128, 127).astype(np.int8)
    return f16_trunc(d), d, q


def quant_i8(x):
    """pack_A_i8 per row: fp32 scale amax/127 (amax floored at 1e-6) and q."""
    x = np.asarray(x, np.float32)
    b = x.reshape(x.shape[0], -1, 32)
    amax = np.maximum(np.abs(b).max(axis=2), F32(1e-6))
    s = (amax / F32(127.0)).astype(np.float32)
    inv = (F32(1.0) / s).astype(np.float32)
    q = np.clip(np.rint(b * inv[..., None]), -128, 127).astype(np.int8)
    return s, q


def quant_q8_K(x):
    """pack_A_q3k per row and 256-block: fp32 scale amax/127 (0 for an all-zero block), q by
    roundf (half away from zero)."""
    x = np.asarray(x, np.float32)
    b = x.reshape(x.shape[0], -1, 256)
    amax = np.abs(b).max(axis=2)
    d = (amax / F32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        rep = np.where(d != 0, F32(1.0) / d, F32(0.0)).astype(np.float32)
    v = (b * rep[..., None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -128, 127).astype(np.int8)
    return d, q


# ------------------------------------------------------------------------------------------------
# weight decoders in the reference's fp32 operation order
# ------------------------------------------------------------------------------------------------
def _k_scale_min(s):
    s = s.astype(np.int64)
    sh = s.shape[:-1] + (8,)
    sc, mn = np.zeros(sh, np.int64), np.zeros(sh, np.int64)
    sc[..., :4], mn[..., :4] = s[..., 0:4] & 63, s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn


def dequant_f32(qtype, W):
    """fp32 values of an (N, blocks) weight, each rounded as the reference's decoder computes it."""
    N, nb = W.shape
    e = np.arange(256)
    if qtype == synth.Q4_0:                        # qwen_moe.c:164-165: (nib - 8) * d
        d = f16_to_f32(W["d"])
        q = np.concatenate([(W["qs"] & 15).astype(np.int64) - 8, (W["qs"] >> 4).astype(np.int64) - 8], axis=2)
        return (q.astype(np.float32) * d[..., None]).reshape(N, nb * 32)
    if qtype == synth.Q8_0:                        # qwen_moe.c:162-163: q * d
        return (W["qs"].astype(np.float32) * f16_to_f32(W["d"])[..., None]).reshape(N, nb * 32)
    if qtype in (synth.Q4_K, synth.Q5_K):          # d1 = d * sc, m1 = dmin * m, d1 * q - m1
        d, dmin = f16_to_f32(W["d"]), f16_to_f32(W["dmin"])
        sc, mn = _k_scale_min(W["scales"])
        sub = e // 32
        d1 = (d[..., None] * sc.astype(np.float32)).astype(np.float32)[..., sub]
        m1 = (dmin[..., None] * mn.astype(np.float32)).astype(np.float32)[..., sub]
        if qtype == synth.Q4_K:
            c, hi, l = e // 64, (e // 32) % 2, e % 32
            q = (W["qs"][..., 32 * c + l].astype(np.int64) >> (4 * hi)) & 15
        else:
            c, hi, l = e // 64, (e // 32) % 2, e % 32
            nib = (W["qs"][..., 32 * c + l].astype(np.int64) >> (4 * hi)) & 15
            q = nib + 16 * ((W["qh"][..., l].astype(np.int64) >> (e // 32)) & 1)
        return (d1 * q.astype(np.float32) - m1).astype(np.float32).reshape(N, nb * 256)
    if qtype == synth.Q3_K:                        # dequantize_q3_K_block: dl = d * (sc - 32); dl * q
        d = f16_to_f32(W["d"])
        s = W["scales"].astype(np.int64)
        i = np.arange(16)
        s6 = ((s[..., i % 8] >> (4 * (i // 8))) & 15) | (((s[..., 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)
        h, j, l = e // 128, (e // 32) % 4, e % 32
        low = (W["qs"][..., 32 * h + l].astype(np.int64) >> (2 * j)) & 3
        hb = (W["hmask"][..., l].astype(np.int64) >> (4 * h + j)) & 1
        q = low - 4 * (1 - hb)
        dl = (d[..., None] * (s6 - 32).astype(np.float32)).astype(np.float32)
        return (dl[..., 8 * h + 2 * j + l // 16] * q.astype(np.float32)).astype(np.float32).reshape(N, nb * 256)
    if qtype == synth.Q6_K:                        # qwen_moe.c:168-177: d * sc * q
        d = f16_to_f32(W["d"])
        h, p = e // 128, e % 128
        low = (W["ql"][..., 64 * h + p % 64].astype(np.int64) >> (4 * (p // 64))) & 15
        top = (W["qh"][..., 32 * h + p % 32].astype(np.int64) >> (2 * (p // 32))) & 3
        q = (low | (top << 4)) - 32
        dsc = (d[..., None] * W["scales"][..., e // 16].astype(np.float32)).astype(np.float32)
        return (dsc * q.astype(np.float32)).astype(np.float32).reshape(N, nb * 256)
    raise ValueError(qtype)


# ------------------------------------------------------------------------------------------------
# GEMVs
# ------------------------------------------------------------------------------------------------
def _block_sums_rowwise(qw, dw, qa, sa, rows=512):
    """bench/vendor_ime_a2_full.c:246-258 / vendor_ime_i8_full.c:183-189 for one activation row:
    y[n] = sum over blocks b (in order) of [fp32 running sum over c of ((qa*sa) * qw) * dw]."""
    N = qw.shape[0]
    y = np.empty(N, np.float32)
    xa = (qa.astype(np.float32) * sa[:, None]).astype(np.float32)           # (nb, 32)
    for r0 in range(0, N, rows):
        p = (xa[None] * qw[r0:r0 + rows].astype(np.float32)).astype(np.float32)
        p = (p * dw[r0:r0 + rows, :, None]).astype(np.float32)
        blk = np.add.accumulate(p, axis=2, dtype=np.float32)[..., -1]       # element order
        y[r0:r0 + rows] = np.add.accumulate(blk, axis=1, dtype=np.float32)[:, -1]
    return y


def gemv_q4_0(W, x):
    """y[M][N] for Q4_0 weights and Q8_0 activations (fp16 scale by truncation)."""
    d16, _, q = quant_q8_0(x)
    qw = np.concatenate([(W["qs"] & 15).astype(np.int8) - 8, (W["qs"] >> 4).astype(np.int8) - 8], axis=2)
    dw = f16_to_f32(W["d"])
    return np.stack([_block_sums_rowwise(qw, dw, q[m], f16_to_f32(d16[m])) for m in range(len(q))])


def requant_q8_0(qtype, W):
    """lin_new_i8 (qwen_moe_q3k.c:872-886): fp32 dequantization, then quantize_q8_0_native per 32;
    returns (fp16 bits of d, q)."""
    N = W.shape[0]
    w = dequant_f32(qtype, W)
    d16, _, q = quant_q8_0(w)
    return d16.reshape(N, -1), q.reshape(N, -1, 32)


def gemv_i8(qtype, W, x):
    """int8 path: requantized weights, pack_A_i8 activations, per-block fp32 sums."""
    d16, qw = requant_q8_0(qtype, W)
    s, q = quant_i8(x)
    dw = f16_to_f32(d16)
    return np.stack([_block_sums_rowwise(qw, dw, q[m], s[m]) for m in range(len(q))])


def gemv_kquant(qtype, W, x, wdeq=None):
    """Q4_K / Q3_K weights and Q8_K activations: fp32-decoded weights times the activation's own
    int8 and scale, accumulated in double (bench/q3k_probe.c:446-456), returned as fp32."""
    if wdeq is None:
        wdeq = dequant_f32(qtype, W)
    d, q = quant_q8_K(x)
    a = q.astype(np.float64) * d.astype(np.float64)[..., None]              # exact products
    a = a.reshape(a.shape[0], -1)
    return (a @ wdeq.astype(np.float64).T).astype(np.float32)


def gemv(qtype, W, x):
    if qtype == synth.Q4_0:
        return gemv_q4_0(W, x)
    if qtype in (synth.Q8_0, synth.Q5_K, synth.Q6_K):
        return gemv_i8(qtype, W, x)
    return gemv_kquant(qtype, W, x)


# ------------------------------------------------------------------------------------------------
# MoE layer
# ------------------------------------------------------------------------------------------------
def expf(x):
    """Correctly rounded binary32 exp (stand-in for libm expf, see the module docstring)."""
    with np.errstate(over="ignore"):                 # overflow to inf, as expf does
        return np.exp(np.asarray(x, np.float32).astype(np.float64)).astype(np.float32)


def route(hn, R, n_act):
    """qwen_moe.c:296-301 per row: logits, probabilities, sel, sw."""
    M = hn.shape[0]
    n_exp = R.shape[0]
    logits = np.empty((M, n_exp), np.float32)
    probs = np.empty((M, n_exp), np.float32)
    sel = np.empty((M, n_act), np.int64)
    sw = np.empty((M, n_act), np.float32)
    for m in range(M):
        prod = (R * hn[m][None]).astype(np.float32)
        rl = np.add.accumulate(prod, axis=1, dtype=np.float32)[:, -1]       # s += rw[i]*hn[i]
        logits[m] = rl
        mx = F32(-1e30)
        for v in rl:
            if v > mx:
                mx = v
        ex = expf((rl - mx).astype(np.float32))
        s = np.add.accumulate(ex, dtype=np.float32)[-1]
        p = (ex * (F32(1.0) / s)).astype(np.float32)
        probs[m] = p
        chosen = []
        for a in range(n_act):
            bi, bv = -1, F32(-1.0)
            for e in range(n_exp):
                if e not in chosen and p[e] > bv:
                    bv, bi = p[e], e
            chosen.append(bi)
            sel[m, a], sw[m, a] = bi, bv
        ssum = np.add.accumulate(sw[m], dtype=np.float32)[-1]
        sw[m] = (sw[m] / ssum).astype(np.float32)
    return logits, probs, sel, sw


def swiglu(g, u):
    """qwen_moe.c:309: g / (1 + expf(-g)) * u in fp32."""
    g = np.asarray(g, np.float32)
    return ((g / (F32(1.0) + expf(-g))).astype(np.float32) * u).astype(np.float32)


def moe_layer(hn, R, Wg, Wu, Wd, n_act, gate_up=None):
    """qwen_moe.c:294-311 for M rows.  gate_up(m, e) -> (g, u) may supply the gate / up
    projections from elsewhere (the tests substitute the oracle's to show that every difference
    beyond tolerance comes from requantizing the activation).  Returns out, sel, sw, probs and
    the per-(row, slot) activations fed to the down projection."""
    M, d = hn.shape
    logits, probs, sel, sw = route(hn, R, n_act)
    cache = {}

    def deq(tag, e, W):
        if (tag, e) not in cache:
            cache[(tag, e)] = dequant_f32(synth.Q4_K, W[e])
        return cache[(tag, e)]

    out = np.zeros((M, d), np.float32)
    acts = np.zeros((M, n_act, Wg.shape[1]), np.float32)
    for m in range(M):
        eout = np.zeros(d, np.float32)
        for a in range(n_act):
            e = int(sel[m, a])
            if gate_up is None:
                g = gemv_kquant(synth.Q4_K, None, hn[m:m + 1], deq("g", e, Wg))[0]
                u = gemv_kquant(synth.Q4_K, None, hn[m:m + 1], deq("u", e, Wu))[0]
            else:
                g, u = gate_up(m, e)
            act = swiglu(g, u)
            acts[m, a] = act
            y = gemv_kquant(synth.Q4_K, None, act[None], deq("d", e, Wd))[0]
            eout = (eout + (sw[m, a] * y).astype(np.float32)).astype(np.float32)
        out[m] = eout
    return out, sel, sw, probs, acts
