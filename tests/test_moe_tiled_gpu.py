"""Tiled expert layout (moe_pack_experts + X100_MOE_TILED): the regrouping against an independent
numpy statement of the layout, and the MoE layer on tiled experts against the same layer on the
ggml-layout experts, bit for bit, on every kernel path (up to 8 rows: persistent gate/up, fused
down in one or two row groups, union-slot down for large ff; 9 or more rows: the matrix-core
kernels, activations in one or two halves), with and without the residual add."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


def tiled_numpy(w, n_exp, rows, K):
    """The layout as a reshape: 16-byte granules (row, super-block, granule) -> (row group,
    super-block, granule, row within the group)."""
    nsb = K // 256
    g = np.ascontiguousarray(w).view(np.uint8).reshape(n_exp, rows // 8, 8, nsb, 9, 16)
    return np.ascontiguousarray(g.transpose(0, 1, 3, 4, 2, 5)).reshape(-1)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1)).to(dev)


def pack_dev(w_dev, n_exp, rows, K, dev):
    import torch
    out = torch.empty_like(w_dev)
    x100hip.moe_pack_experts(n_exp, rows, K, w_dev.data_ptr(), out.data_ptr(),
                             torch.cuda.current_stream().cuda_stream)
    return out


_cache = {}


def layer(n_exp, d, ff, seed, dev):
    import torch
    key = (n_exp, d, ff, seed)
    if key not in _cache:
        Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed)
        R = synth.moe_router(n_exp, d, seed + 1)
        gg = [to_dev(w, dev) for w in (Wg, Wu, Wd)]
        tl = [pack_dev(gg[0], n_exp, ff, d, dev), pack_dev(gg[1], n_exp, ff, d, dev),
              pack_dev(gg[2], n_exp, d, ff, dev)]
        _cache.clear()
        _cache[key] = (Wg, Wu, Wd, R, gg, tl, torch.from_numpy(R).to(dev))
    return _cache[key]


def run(hn, L, n_act, dev, tiled, out0=None, residual=False):
    import torch
    Wg, Wu, Wd, R, gg, tl, dR = L
    M, d = hn.shape
    n_exp, ff = Wg.shape[0], Wg.shape[1]
    W = tl if tiled else gg
    dh = torch.from_numpy(hn).to(dev)
    out = torch.from_numpy(out0.copy()).to(dev) if out0 is not None else torch.full((M, d), float("nan"), device=dev)
    sel = torch.full((M, n_act), -1, dtype=torch.int32, device=dev)
    sw = torch.zeros((M, n_act), dtype=torch.float32, device=dev)
    x100hip.moe_layer(M, d, ff, n_exp, n_act, dh.data_ptr(), dR.data_ptr(), W[0].data_ptr(), W[1].data_ptr(),
                      W[2].data_ptr(), out.data_ptr(), residual, sel.data_ptr(), sw.data_ptr(),
                      torch.cuda.current_stream().cuda_stream, tiled=tiled)
    torch.cuda.synchronize()
    return out.cpu().numpy(), sel.cpu().numpy(), sw.cpu().numpy()


@pytest.mark.parametrize("n_exp,rows,K", [(3, 8, 256), (2, 24, 768), (5, 16, 4096), (128, 768, 2048)])
def test_pack_matches_the_layout(dev, n_exp, rows, K):
    import torch
    rng = np.random.default_rng(rows + K)
    w = rng.integers(0, 256, n_exp * rows * (K // 256) * 144, dtype=np.uint8)
    got = pack_dev(to_dev(w, dev), n_exp, rows, K, dev)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), tiled_numpy(w, n_exp, rows, K))


def test_pack_rejects_bad_arguments(dev):
    import torch
    buf = torch.zeros(2 * 16 * 144 * 2, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    for args in [(1, 12, 256), (1, 8, 200), (0, 8, 256)]:   # rows % 8, K % 256, no expert
        with pytest.raises(x100hip.X100Error):
            x100hip.moe_pack_experts(*args, buf.data_ptr(), buf[2304:].data_ptr(), s)
    with pytest.raises(x100hip.X100Error):                   # in place
        x100hip.moe_pack_experts(1, 16, 256, buf.data_ptr(), buf[16:].data_ptr(), s)


CASES = [
    # (M, n_exp, d, ff, n_act): the Qwen3-30B-A3B layer on both paths
    (1, 128, 2048, 768, 8), (2, 128, 2048, 768, 8), (4, 128, 2048, 768, 8), (5, 128, 2048, 768, 8),
    (7, 128, 2048, 768, 8), (8, 128, 2048, 768, 8), (9, 128, 2048, 768, 8), (33, 128, 2048, 768, 8),
    (64, 128, 2048, 768, 8),
    # small shapes, few and many rows
    (3, 16, 512, 256, 4), (4, 200, 256, 256, 6), (17, 64, 1024, 512, 2), (100, 8, 256, 256, 8),
    # ff of 16 super-blocks: union-slot down (few rows), two activation halves (matrix cores)
    (3, 16, 512, 4096, 8), (6, 16, 512, 4096, 8), (8, 16, 512, 4096, 4), (12, 16, 512, 4096, 4),
    # d = ff = 4096
    (3, 4, 4096, 4096, 2), (16, 4, 4096, 4096, 2),
]


@pytest.mark.parametrize("M,n_exp,d,ff,n_act", CASES)
def test_tiled_layer_equals_ggml_layout(dev, M, n_exp, d, ff, n_act):
    L = layer(n_exp, d, ff, 900 + n_exp + d // 256, dev)
    hn = synth.normal_f32(950 + M, (M, d))
    a, sa, wa = run(hn, L, n_act, dev, tiled=False)
    b, sb, wb = run(hn, L, n_act, dev, tiled=True)
    assert np.array_equal(sa, sb)
    assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "%d elements differ" % int(
        (a.view(np.uint32) != b.view(np.uint32)).sum())


@pytest.mark.parametrize("M", [2, 12])
def test_tiled_layer_residual_against_the_oracle(dev, M):
    L = layer(128, 2048, 768, 910, dev)
    Wg, Wu, Wd, R = L[:4]
    hn = synth.normal_f32(960 + M, (M, 2048))
    out0 = synth.normal_f32(961 + M, (M, 2048))
    got, gsel, _ = run(hn, L, 8, dev, tiled=True, out0=out0, residual=True)
    ref, rsel, _ = ol.moe_layer(hn, R, Wg, Wu, Wd, 8, out=out0.copy(), residual=True)
    assert np.array_equal(gsel, rsel)
    err = np.abs(got - ref)
    assert not (err > ATOL + RTOL * np.abs(ref)).any()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_unknown_flag_rejected(dev):
    import torch
    L = layer(16, 512, 256, 920, dev)
    hn = torch.zeros((2, 512), device=dev)
    out = torch.zeros((2, 512), device=dev)
    W = L[5]
    rc = x100hip.lib().moe_layer_hip(2, 512, 256, 16, 4, hn.data_ptr(), L[6].data_ptr(), W[0].data_ptr(),
                                     W[1].data_ptr(), W[2].data_ptr(), out.data_ptr(), 4, None, None,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == x100hip.X100_EINVAL
