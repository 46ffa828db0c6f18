"""One Qwen3-MoE decoder layer on the GPU (x100_decode.h) against the oracle's layer
(orc_attn_decode / orc_decode_layer), which sums in the kernels' orders: h after the attention
half and after the whole layer, the KV-cache rows written at pos, the experts and their weights
all bit for bit; every other cache row untouched."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip
from test_decode_oracle import TYPES, caches, make_cfg

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


class GpuLayer:
    def __init__(self, cfg, L, types, dev):
        import torch
        self.cfg, self.dev = cfg, dev
        s = torch.cuda.current_stream().cuda_stream
        self.keep = []

        def f32(a):
            t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
            self.keep.append(t)
            return t.data_ptr()

        def packed(qt, W):
            N, K = W.shape[0], W.shape[1] * synth.BLOCK_ELEMS[qt]
            raw = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
            pk = torch.empty(x100hip.packed_bytes(qt, N, K), dtype=torch.uint8, device=dev)
            x100hip.pack(qt, N, K, raw.data_ptr(), pk.data_ptr(), s)
            self.keep += [raw, pk]
            return pk.data_ptr()

        def raw(W):
            t = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
            self.keep.append(t)
            return t.data_ptr()

        self.kc = torch.zeros((cfg.n_head_kv, cfg.ctx, cfg.head_dim), dtype=torch.float32, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.w = x100hip.LayerWeights(
            f32(L["attn_norm"]), f32(L["q_norm"]), f32(L["k_norm"]), f32(L["ffn_norm"]), packed(types[0], L["wq"]),
            packed(types[1], L["wk"]), packed(types[2], L["wv"]), packed(types[3], L["wo"]), f32(L["router"]),
            raw(L["wg"]), raw(L["wu"]), raw(L["wd"]), self.kc.data_ptr(), self.vc.data_ptr())
        self.gcfg = x100hip.LayerCfg(*[getattr(cfg, n) for n, _ in x100hip.LayerCfg._fields_])
        torch.cuda.synchronize()

    def set_cache(self, kc, vc):
        import torch
        self.kc.copy_(torch.from_numpy(kc))
        self.vc.copy_(torch.from_numpy(vc))

    def run(self, pos, h, whole=False):
        import torch
        s = torch.cuda.current_stream().cuda_stream
        dh = torch.from_numpy(h.copy()).to(self.dev)
        sel = torch.full((self.cfg.n_act,), -1, dtype=torch.int32, device=self.dev)
        sw = torch.zeros((self.cfg.n_act,), dtype=torch.float32, device=self.dev)
        if whole:
            x100hip.decode_layer(self.gcfg, self.w, pos, dh.data_ptr(), sel.data_ptr(), sw.data_ptr(), s)
        else:
            x100hip.attn_decode(self.gcfg, self.w, pos, dh.data_ptr(), s)
        torch.cuda.synchronize()
        return dh.cpu().numpy(), sel.cpu().numpy(), sw.cpu().numpy()


def close(got, ref, what):
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), "%s: %d outside tolerance, max err %g" % (what, int(bad.sum()), float(err.max()))
    assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(ref).view(np.uint32)), \
        "%s: not bit-identical (max err %g)" % (what, float(err.max()))


def check_attn(cfg, types, L, pos, seed, dev, gl=None):
    gl = gl or GpuLayer(cfg, L, types, dev)
    kc, vc = caches(cfg, pos, seed)
    gl.set_cache(kc, vc)
    h = synth.normal_f32(seed + 5, (cfg.d,))
    got, _, _ = gl.run(pos, h)
    rh, rk, rv = h.copy(), kc.copy(), vc.copy()
    ol.attn_decode(cfg, L, rk, rv, pos, rh)
    close(got, rh, "h pos %d" % pos)
    gk, gv = gl.kc.cpu().numpy(), gl.vc.cpu().numpy()
    close(gk[:, pos], rk[:, pos], "k row")
    close(gv[:, pos], rv[:, pos], "v row")
    mask = np.ones(cfg.ctx, bool)
    mask[pos] = False
    assert np.array_equal(gk[:, mask], kc[:, mask]) and np.array_equal(gv[:, mask], vc[:, mask])
    return gl


def test_attn_decode_positions(dev):
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=100)
    gl = None
    for pos in (0, 1, 17, 39):
        gl = check_attn(cfg, TYPES, L, pos, 200 + pos, dev, gl)


@pytest.mark.parametrize("nh,nkv", [(16, 2), (16, 1), (8, 8)])
def test_attn_decode_gqa_groups(dev, nh, nkv):
    types = (synth.Q4_K,) * 4
    cfg = make_cfg(types, n_head=nh, n_head_kv=nkv, ctx=300)
    L = synth.decode_layer_weights(512, nh, nkv, 128, 256, 8, types, seed=110 + nh + nkv)
    gl = None
    for pos in (0, 5, 130, 299):
        gl = check_attn(cfg, types, L, pos, 300 + pos, dev, gl)


def test_decode_steps_from_empty_cache(dev):
    # six tokens in a row, each layer call reading what the previous ones wrote
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=120)
    gl = GpuLayer(cfg, L, TYPES, dev)
    rk = np.zeros((cfg.n_head_kv, cfg.ctx, cfg.head_dim), np.float32)
    rv = np.zeros_like(rk)
    for pos in range(6):
        h = synth.normal_f32(400 + pos, (cfg.d,))
        got, _, _ = gl.run(pos, h)
        rh = h.copy()
        ol.attn_decode(cfg, L, rk, rv, pos, rh)
        close(got, rh, "step %d" % pos)
        close(gl.kc.cpu().numpy()[:, :pos + 1], rk[:, :pos + 1], "k cache step %d" % pos)


def test_attn_decode_qwen3_shape_long_context(dev):
    # Qwen3-30B-A3B attention: d 2048, 32 query heads, 4 KV heads, head_dim 128; 4096 positions
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    cfg = make_cfg(types, d=2048, n_head=32, n_head_kv=4, ctx=4096)
    L = synth.decode_layer_weights(2048, 32, 4, 128, 256, 8, types, seed=130)
    gl = None
    # chunks of 16, 24, 32, 40 and 64 positions (2 to 8 steps of 8 positions per block)
    for pos in (1000, 1300, 2000, 2500, 4095):
        gl = check_attn(cfg, types, L, pos, 500 + pos, dev, gl)


def test_attn_decode_qwen3_shape_8192_positions(dev):
    # 128 positions per chunk (16 steps of 8 positions per block)
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    cfg = make_cfg(types, d=2048, n_head=32, n_head_kv=4, ctx=8192)
    L = synth.decode_layer_weights(2048, 32, 4, 128, 256, 8, types, seed=135)
    gl = None
    for pos in (5000, 8191):
        gl = check_attn(cfg, types, L, pos, 900 + pos, dev, gl)


def test_decode_layer_qwen3_30b_a3b(dev):
    """The whole layer at the Qwen3-30B-A3B shape with its mixed weight types."""
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    cfg = make_cfg(types, d=2048, n_head=32, n_head_kv=4, ff=768, n_exp=128, n_act=8, ctx=1024)
    L = synth.decode_layer_weights(2048, 32, 4, 128, 768, 128, types, seed=140)
    gl = GpuLayer(cfg, L, types, dev)
    for pos in (0, 700, 1023):
        kc, vc = caches(cfg, pos, 600 + pos)
        h = synth.normal_f32(610 + pos, (cfg.d,))
        gl.set_cache(kc, vc)
        got, gsel, gsw = gl.run(pos, h, whole=True)
        rh, rk, rv = h.copy(), kc.copy(), vc.copy()
        rsel, rsw = ol.decode_layer(cfg, L, rk, rv, pos, rh)
        assert np.array_equal(gsel, rsel)
        close(gsw, rsw, "router weights pos %d" % pos)
        close(got, rh, "layer pos %d" % pos)
        close(gl.kc.cpu().numpy()[:, pos], rk[:, pos], "k row")
        close(gl.vc.cpu().numpy()[:, pos], rv[:, pos], "v row")


@pytest.mark.parametrize("types,n_exp,n_act,ff", [
    ((synth.Q4_K, synth.Q4_K, synth.Q4_K, synth.Q4_0), 33, 3, 512),   # odd expert count: a block holds a
    ((synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K), 9, 8, 256),     # router and a quantizer wave
    ((synth.Q4_0, synth.Q8_0, synth.Q4_0, synth.Q4_K), 64, 1, 1024),
])
def test_decode_layer_d2048_moe_variants(dev, types, n_exp, n_act, ff):
    """Whole layers at d = 2048 (where the step before the MoE block, h += o and its RMSNorm, runs
    inside the MoE router kernel) with other expert counts, slot counts, ff and weight types."""
    cfg = make_cfg(types, d=2048, n_head=16, n_head_kv=4, ff=ff, n_exp=n_exp, n_act=n_act, ctx=256)
    L = synth.decode_layer_weights(2048, 16, 4, 128, ff, n_exp, types, seed=170 + n_exp)
    gl = GpuLayer(cfg, L, types, dev)
    for pos in (0, 255):
        kc, vc = caches(cfg, pos, 700 + pos + n_exp)
        h = synth.normal_f32(710 + pos + n_exp, (cfg.d,)) * np.float32(1 + pos % 7)
        gl.set_cache(kc, vc)
        got, gsel, gsw = gl.run(pos, h, whole=True)
        rh, rk, rv = h.copy(), kc.copy(), vc.copy()
        rsel, rsw = ol.decode_layer(cfg, L, rk, rv, pos, rh)
        assert np.array_equal(gsel, rsel)
        close(gsw, rsw, "router weights pos %d" % pos)
        close(got, rh, "layer pos %d" % pos)


def test_decode_layer_unaligned_h(dev):
    """h 4 bytes past a 16-byte boundary: the layer takes the unfolded norm launches (the folded
    norms load h as float4) and still matches the oracle bit for bit."""
    import torch
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    cfg = make_cfg(types, d=2048, n_head=32, n_head_kv=4, ff=768, n_exp=128, n_act=8, ctx=64)
    L = synth.decode_layer_weights(2048, 32, 4, 128, 768, 128, types, seed=190)
    gl = GpuLayer(cfg, L, types, dev)
    pos = 40
    kc, vc = caches(cfg, pos, 800)
    h = synth.normal_f32(801, (cfg.d,))
    gl.set_cache(kc, vc)
    buf = torch.zeros(cfg.d + 4, dtype=torch.float32, device=dev)
    buf[1:cfg.d + 1] = torch.from_numpy(h).to(dev)
    sel = torch.full((cfg.n_act,), -1, dtype=torch.int32, device=dev)
    sw = torch.zeros((cfg.n_act,), dtype=torch.float32, device=dev)
    assert (buf.data_ptr() + 4) % 16 == 4
    x100hip.decode_layer(gl.gcfg, gl.w, pos, buf.data_ptr() + 4, sel.data_ptr(), sw.data_ptr(),
                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    rh, rk, rv = h.copy(), kc.copy(), vc.copy()
    rsel, rsw = ol.decode_layer(cfg, L, rk, rv, pos, rh)
    assert np.array_equal(sel.cpu().numpy(), rsel)
    close(sw.cpu().numpy(), rsw, "router weights")
    close(got[1:cfg.d + 1], rh, "layer")
    assert got[0] == 0 and not got[cfg.d + 1:].any()
    close(gl.kc.cpu().numpy()[:, pos], rk[:, pos], "k row")


def test_decode_rejects_bad_configs(dev):
    cfg = make_cfg()
    L = synth.decode_layer_weights(512, 4, 2, 128, 256, 8, TYPES, seed=150)
    gl = GpuLayer(cfg, L, TYPES, dev)
    import torch
    dh = torch.zeros(512, device=dev)
    for bad in (dict(pos=cfg.ctx), dict(pos=-1), dict(head_dim=64), dict(n_head=3), dict(wq_type=99)):
        c = x100hip.LayerCfg(*[getattr(gl.gcfg, n) for n, _ in x100hip.LayerCfg._fields_])
        pos = bad.pop("pos", 0)
        for k, v in bad.items():
            setattr(c, k, v)
        with pytest.raises(x100hip.X100Error):
            x100hip.attn_decode(c, gl.w, pos, dh.data_ptr())
