"""The oracle's decode step (rmsnorm, rope, attention half, whole layer; qwen_moe.c:187-189, 278-311)
against closed forms, invariants and an independent float64 numpy restatement."""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol
import synth


def test_rmsnorm_closed_form():
    x = synth.normal_f32(1, (2048,))
    w = synth.normal_f32(2, (2048,))
    got = ol.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)
    # a constant row c: every element w * c / sqrt(c^2 + eps)
    c = np.full(256, 3.0, np.float32)
    np.testing.assert_allclose(ol.rmsnorm(c, np.ones(256, np.float32), 0.0), np.ones(256), rtol=1e-7)


def np_rope(v, pos, base):
    hd = v.size
    i = np.arange(hd // 2)
    e = (np.float32(-2.0) * i.astype(np.float32) / np.float32(hd)).astype(np.float32)
    fr = np.power(np.float64(base), e.astype(np.float64)).astype(np.float32)
    a = (np.float32(pos) * fr).astype(np.float32).astype(np.float64)
    x, y = v[:hd // 2].astype(np.float64), v[hd // 2:].astype(np.float64)
    return np.concatenate([x * np.cos(a) - y * np.sin(a), x * np.sin(a) + y * np.cos(a)])


@pytest.mark.parametrize("pos", [0, 1, 7, 1000, 40959])
def test_rope(pos):
    hd, base = 128, 1e6
    c, s = ol.rope_table(hd, pos, base)
    if pos == 0:
        assert np.all(c == 1.0) and np.all(s == 0.0)
    v = synth.normal_f32(10 + pos, (hd,))
    got = v.copy()
    ol.oracle().orc_rope_apply(ol._p(got), hd, ol._p(c), ol._p(s))
    np.testing.assert_allclose(got, np_rope(v, pos, base), rtol=1e-5, atol=1e-6)
    # each (i, i + hd/2) pair is rotated: its length is kept
    n0 = v[:64] ** 2 + v[64:] ** 2
    n1 = got[:64].astype(np.float64) ** 2 + got[64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    # frequency 0 (i = 0) turns by exactly pos radians
    np.testing.assert_allclose(c[0], np.cos(np.float64(pos)), atol=1e-7)


CFG = dict(d=512, n_head=4, n_head_kv=2, head_dim=128, ff=256, n_exp=8, n_act=4, ctx=40, eps=1e-6,
           rope_base=1e6)
TYPES = (synth.Q3_K, synth.Q8_0, synth.Q4_0, synth.Q5_K)


def make_cfg(types=TYPES, **kw):
    c = dict(CFG)
    c.update(kw)
    return ol.LayerCfg(c["d"], c["n_head"], c["n_head_kv"], c["head_dim"], c["ff"], c["n_exp"], c["n_act"], c["ctx"],
                       c["eps"], c["rope_base"], *types)


def caches(cfg, pos, seed):
    shape = (cfg.n_head_kv, cfg.ctx, cfg.head_dim)
    kc = np.zeros(shape, np.float32)
    vc = np.zeros(shape, np.float32)
    kc[:, :pos] = synth.normal_f32(seed, (cfg.n_head_kv, pos, cfg.head_dim))
    vc[:, :pos] = synth.normal_f32(seed + 1, (cfg.n_head_kv, pos, cfg.head_dim))
    return kc, vc


def np_attn(cfg, L, kc, vc, pos, h, types=TYPES):
    """The attention half in float64 numpy (GEMVs through the oracle's qgemv, which test_oracle pins)."""
    hd, nh, nkv = cfg.head_dim, cfg.n_head, cfg.n_head_kv
    hn = ol.rmsnorm(h, L["attn_norm"], cfg.eps)
    q = ol.qgemv(types[0], L["wq"], hn[None])[0].astype(np.float64).reshape(nh, hd)
    k = ol.qgemv(types[1], L["wk"], hn[None])[0].astype(np.float64).reshape(nkv, hd)
    v = ol.qgemv(types[2], L["wv"], hn[None])[0].reshape(nkv, hd)

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + cfg.eps) * w

    q = np.stack([np_rope(r.astype(np.float32), pos, cfg.rope_base) for r in norm(q, L["q_norm"]).astype(np.float32)])
    k = np.stack([np_rope(r.astype(np.float32), pos, cfg.rope_base) for r in norm(k, L["k_norm"]).astype(np.float32)])
    K = kc.astype(np.float64).copy()
    V = vc.astype(np.float64).copy()
    K[:, pos] = k
    V[:, pos] = v
    gpr = nh // nkv
    att = np.zeros((nh, hd))
    for hh in range(nh):
        s = K[hh // gpr, :pos + 1] @ q[hh] / np.sqrt(hd)
        p = np.exp(s - s.max())
        att[hh] = (p / p.sum()) @ V[hh // gpr, :pos + 1]
    o = ol.qgemv(types[3], L["wo"], att.reshape(1, -1).astype(np.float32))[0]
    return h.astype(np.float64) + o, K, V


@pytest.mark.parametrize("pos", [0, 1, 17, 39])
def test_attn_decode_vs_numpy(pos):
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=100)
    kc, vc = caches(cfg, pos, 200 + pos)
    h = synth.normal_f32(300 + pos, (512,))
    ref_h, K, V = np_attn(cfg, L, kc, vc, pos, h)
    h2, kc2, vc2 = h.copy(), kc.copy(), vc.copy()
    ol.attn_decode(cfg, L, kc2, vc2, pos, h2)
    np.testing.assert_allclose(h2, ref_h, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(kc2, K, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(vc2, V, rtol=1e-6, atol=0)
    mask = np.ones(cfg.ctx, bool)
    mask[pos] = False
    assert np.array_equal(kc2[:, mask], kc[:, mask]) and np.array_equal(vc2[:, mask], vc[:, mask])


def test_attn_position_zero_is_the_value_row():
    # one position: softmax = 1, each head's output is its KV head's v, so h += Wo.(v repeated)
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=101)
    kc, vc = caches(cfg, 0, 1)
    h = synth.normal_f32(5, (512,))
    h2 = h.copy()
    ol.attn_decode(cfg, L, kc, vc, 0, h2)
    v = vc[:, 0]
    att = np.concatenate([v[hh // 2] for hh in range(4)])
    o = ol.qgemv(TYPES[3], L["wo"], att[None])[0]
    np.testing.assert_allclose(h2, h + o, rtol=1e-6, atol=1e-6)


def test_decode_layer_is_attention_then_moe():
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=102)
    kc, vc = caches(cfg, 9, 3)
    h = synth.normal_f32(6, (512,))
    h1, kc1, vc1 = h.copy(), kc.copy(), vc.copy()
    sel, sw = ol.decode_layer(cfg, L, kc1, vc1, 9, h1)
    h2, kc2, vc2 = h.copy(), kc.copy(), vc.copy()
    ol.attn_decode(cfg, L, kc2, vc2, 9, h2)
    hn = ol.rmsnorm(h2, L["ffn_norm"], cfg.eps)
    out, rsel, rsw = ol.moe_layer(hn[None], L["router"], L["wg"], L["wu"], L["wd"], cfg.n_act, out=h2[None].copy(),
                                  residual=True)
    assert np.array_equal(h1.view(np.uint32), out[0].view(np.uint32))
    assert np.array_equal(sel, rsel[0]) and np.array_equal(sw, rsw[0])
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
