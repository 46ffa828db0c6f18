"""Whole decoder layers on seeded random shapes against the oracle's layer, bit for bit: d from 512
to 4096 (at d = 2048 the attention norm and the norm before the MoE block run inside the
projection and router launches), 2 to 32 query heads in GQA groups of 1 to 16, every attention
weight type, 2 to 64 experts with 1 to 8 slots, and positions anywhere in contexts of up to 1500."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
from test_decode_gpu import GpuLayer, close
from test_decode_oracle import caches, make_cfg

pytestmark = pytest.mark.gpu

WTYPES = [synth.Q4_0, synth.Q8_0, synth.Q3_K, synth.Q4_K, synth.Q5_K, synth.Q6_K]


def shapes(seed=4242, n=12):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([512, 1024, 2048, 2048, 3072, 4096]))
        nkv = int(rng.choice([1, 2, 4]))
        gpr = int(rng.choice([1, 2, 4, 8, 16]))
        nh = max(2, min(32, nkv * gpr))
        nh -= nh % nkv
        nh += nh % 2   # Wo's K = 128 n_head a multiple of 256 for the K-quant types
        if nh % nkv:
            nkv = 1
        if i % 3 == 0:   # the Qwen3 checkpoint's mix (q and v one K-quant type, k on the int8 path)
            qt = int(rng.choice([synth.Q3_K, synth.Q4_K]))
            types = (qt, int(rng.choice([synth.Q8_0, synth.Q5_K, synth.Q6_K])), qt, int(rng.choice(WTYPES)))
        else:
            types = tuple(int(rng.choice(WTYPES)) for _ in range(4))
        n_act = int(rng.integers(1, 9))
        n_exp = int(rng.choice([n_act, n_act + 1, 16, 33, 64]))
        ff = int(rng.choice([256, 512]))
        ctx = int(rng.integers(8, 1500))
        pos = int(rng.integers(0, ctx))
        out.append((d, nh, nkv, types, n_exp, n_act, ff, ctx, pos, int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("d,nh,nkv,types,n_exp,n_act,ff,ctx,pos,seed", shapes())
def test_decode_layer_random_shape(dev, d, nh, nkv, types, n_exp, n_act, ff, ctx, pos, seed):
    cfg = make_cfg(types, d=d, n_head=nh, n_head_kv=nkv, ff=ff, n_exp=n_exp, n_act=n_act, ctx=ctx)
    L = synth.decode_layer_weights(d, nh, nkv, 128, ff, n_exp, types, seed=seed % 100000)
    gl = GpuLayer(cfg, L, types, dev)
    kc, vc = caches(cfg, pos, seed % 1000 + 1)
    h = synth.normal_f32(seed % 1000 + 7, (d,))
    gl.set_cache(kc, vc)
    got, gsel, gsw = gl.run(pos, h, whole=True)
    rh, rk, rv = h.copy(), kc.copy(), vc.copy()
    rsel, rsw = ol.decode_layer(cfg, L, rk, rv, pos, rh)
    assert np.array_equal(gsel, rsel)
    close(gsw, rsw, "router weights")
    close(got, rh, "layer")
    close(gl.kc.cpu().numpy()[:, pos], rk[:, pos], "k row")
    close(gl.vc.cpu().numpy()[:, pos], rv[:, pos], "v row")
