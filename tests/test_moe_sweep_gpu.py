"""MoE layer on seeded random shapes (1-12 token rows, 1-8 slots, 1-256 experts, d and ff from 256
to 4096, ggml or tiled experts, with and without the residual add) against the oracle, bit for
bit: the few-row kernels (fused down in one or two row groups, union-slot down for large ff) and
the matrix-core path from 9 rows, on shapes the fixed cases do not name."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu


def shapes(seed=2026, n=24):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 13))
        n_act = int(rng.integers(1, 9))
        n_exp = max(n_act, int(rng.choice([n_act, n_act + 1, 8, 16, 33, 64, 128, 200, 256])))
        d = int(rng.choice([256, 512, 768, 1024, 2048, 3072, 4096]))
        ff = int(rng.choice([256, 512, 768, 1024, 2048, 4096]))
        if d * ff * n_exp > 2048 * 768 * 256:   # keeps the oracle and the weights small
            ff = 256
        out.append((M, n_exp, d, ff, n_act, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)),
                    int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("M,n_exp,d,ff,n_act,residual,tiled,seed", shapes())
def test_moe_random_shape(dev, M, n_exp, d, ff, n_act, residual, tiled, seed):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed)
    R = synth.moe_router(n_exp, d, seed + 1)
    hn = synth.normal_f32(seed + 2, (M, d))
    out0 = synth.normal_f32(seed + 3, (M, d))
    W = [torch.from_numpy(np.ascontiguousarray(w).view(np.uint8).reshape(-1)).to(dev) for w in (Wg, Wu, Wd)]
    if tiled:
        T = [torch.empty_like(w) for w in W]
        for k, (rows, K) in enumerate(((ff, d), (ff, d), (d, ff))):
            x100hip.moe_pack_experts(n_exp, rows, K, W[k].data_ptr(), T[k].data_ptr(), s)
        W = T
    dR, dh = torch.from_numpy(R).to(dev), torch.from_numpy(hn).to(dev)
    out = torch.from_numpy(out0.copy()).to(dev) if residual else torch.full((M, d), float("nan"), device=dev)
    sel = torch.full((M, n_act), -1, dtype=torch.int32, device=dev)
    sw = torch.zeros((M, n_act), dtype=torch.float32, device=dev)
    x100hip.moe_layer(M, d, ff, n_exp, n_act, dh.data_ptr(), dR.data_ptr(), W[0].data_ptr(), W[1].data_ptr(),
                      W[2].data_ptr(), out.data_ptr(), residual, sel.data_ptr(), sw.data_ptr(), s, tiled=tiled)
    torch.cuda.synchronize()
    got, gsel, gsw = out.cpu().numpy(), sel.cpu().numpy(), sw.cpu().numpy()
    ref, rsel, rsw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act, out=out0.copy() if residual else None,
                                  residual=residual)
    assert np.array_equal(gsel, rsel)
    assert np.array_equal(gsw.view(np.uint32), rsw.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "%d elements differ" % int(
        (got.view(np.uint32) != ref.view(np.uint32)).sum())
