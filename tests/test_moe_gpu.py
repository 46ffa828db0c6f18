"""MoE decode layer on the GPU against the oracle MoE block (rel 1e-3 / abs 1e-4 in fp32),
identical expert selection, and the top-k margin at the fixed seeds."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4

_cache = {}


def layer(n_exp, d, ff, seed, dev):
    import torch
    key = (n_exp, d, ff, seed)
    if key not in _cache:
        Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed)
        R = synth.moe_router(n_exp, d, seed + 1)
        dW = [torch.from_numpy(np.ascontiguousarray(w).view(np.uint8).reshape(-1)).to(dev) for w in (Wg, Wu, Wd)]
        _cache.clear()
        _cache[key] = (Wg, Wu, Wd, R, dW, torch.from_numpy(R).to(dev))
    return _cache[key]


def gpu_moe(hn, L, n_act, dev, out0=None, residual=False):
    import torch
    Wg, Wu, Wd, R, dW, dR = L
    M, d = hn.shape
    n_exp, ff = Wg.shape[0], Wg.shape[1]
    s = torch.cuda.current_stream().cuda_stream
    dh = torch.from_numpy(hn).to(dev)
    out = torch.from_numpy(out0.copy()).to(dev) if out0 is not None else torch.full((M, d), float("nan"), device=dev)
    sel = torch.full((M, n_act), -1, dtype=torch.int32, device=dev)
    sw = torch.zeros((M, n_act), dtype=torch.float32, device=dev)
    x100hip.moe_layer(M, d, ff, n_exp, n_act, dh.data_ptr(), dR.data_ptr(), dW[0].data_ptr(),
                      dW[1].data_ptr(), dW[2].data_ptr(), out.data_ptr(), residual, sel.data_ptr(),
                      sw.data_ptr(), s)
    torch.cuda.synchronize()
    return out.cpu().numpy(), sel.cpu().numpy(), sw.cpu().numpy()


def topk_margin(hn, R, n_act):
    if n_act >= R.shape[0]:
        return float("inf")
    logits, _, _ = ol.moe_route(hn, R, n_act)
    srt = -np.sort(-logits, axis=1)
    return float((srt[:, n_act - 1] - srt[:, n_act]).min())


def check(M, n_exp, d, ff, n_act, seed, dev, residual=False):
    L = layer(n_exp, d, ff, seed, dev)
    Wg, Wu, Wd, R = L[:4]
    hn = synth.normal_f32(seed + 2 + M, (M, d))
    out0 = synth.normal_f32(seed + 3, (M, d)) if residual else None
    got, gsel, gsw = gpu_moe(hn, L, n_act, dev, out0, residual)
    ref, rsel, rsw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act, out=None if out0 is None else out0.copy(),
                                  residual=residual)
    margin = topk_margin(hn, R, n_act)
    print("M=%d n_exp=%d d=%d ff=%d: top-%d logit margin %.3g, union %d experts" % (
        M, n_exp, d, ff, n_act, margin, len(set(rsel.ravel().tolist()))))
    assert np.array_equal(gsel, rsel)
    np.testing.assert_allclose(gsw, rsw, rtol=1e-5, atol=1e-7)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), "%d outside tolerance, max rel %g" % (int(bad.sum()), float((err / (np.abs(ref) + 1e-30)).max()))
    # the kernels follow the oracle's operation order throughout: identical bits expected
    assert np.array_equal(gsw.view(np.uint32), rsw.view(np.uint32)), "router weights not bit-identical"
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "%d elements not bit-identical" % int(
        (got.view(np.uint32) != ref.view(np.uint32)).sum())
    return got, ref


@pytest.mark.parametrize("M", [1, 4])
def test_moe_qwen3_30b_a3b_shape(dev, M):
    check(M, 128, 2048, 768, 8, seed=500, dev=dev)


def test_moe_m8_and_residual(dev):
    check(8, 128, 2048, 768, 8, seed=500, dev=dev, residual=True)


@pytest.mark.parametrize("M", [5, 6, 7])
def test_moe_five_to_seven_rows_qwen3_shape(dev, M):
    # above 4 rows: two routing rows per wave, up to 56 union slots, and the fused down projection
    # in two row groups of at most 32 pairs (7 rows: groups of 4 and 3)
    check(M, 128, 2048, 768, 8, seed=540 + M, dev=dev)


@pytest.mark.parametrize("M,n_exp,d,ff,n_act", [(1, 16, 512, 256, 4), (3, 16, 512, 256, 4),
                                                (2, 8, 256, 512, 8), (5, 64, 1024, 512, 2),
                                                (4, 200, 256, 256, 6),
                                                # odd router-wave counts: a router block that also
                                                # holds a quantizer wave
                                                (1, 9, 256, 256, 4), (3, 15, 512, 256, 4)])
def test_moe_small_shapes(dev, M, n_exp, d, ff, n_act):
    check(M, n_exp, d, ff, n_act, seed=600 + M + n_exp, dev=dev)


def test_moe_repeat_calls_stable(dev):
    # every kernel writes the scratch it reads within the call: repeated calls give the same bits
    L = layer(16, 512, 256, 700, dev)
    hn = synth.normal_f32(701, (2, 512))
    a = gpu_moe(hn, L, 4, dev)[0]
    for _ in range(3):
        assert np.array_equal(gpu_moe(hn, L, 4, dev)[0], a)


@pytest.mark.parametrize("M", [2, 4, 8])
def test_moe_batched_rows_equal_single_rows(dev, M):
    # Several token rows (union grouping, fused down in one or two row groups) must give every
    # row exactly what a one-row call gives it (per-row routing and Q8_K quantization)
    L = layer(128, 2048, 768, 500, dev)
    hn = synth.normal_f32(800 + M, (M, 2048))
    out, sel, sw = gpu_moe(hn, L, 8, dev)
    for m in range(M):
        o1, s1, w1 = gpu_moe(hn[m:m + 1], L, 8, dev)
        assert np.array_equal(sel[m], s1[0])
        assert np.array_equal(sw[m].view(np.uint32), w1[0].view(np.uint32))
        assert np.array_equal(out[m].view(np.uint32), o1[0].view(np.uint32)), "row %d differs" % m


# ---- 9 or more token rows: routing per 8-row chunk, pairs grouped by expert into chunks of 32 on
# the matrix cores ----
@pytest.mark.parametrize("M", [9, 12, 15, 16, 64, 512])
def test_moe_many_rows_qwen3_shape(dev, M):
    check(M, 128, 2048, 768, 8, seed=510 + M, dev=dev)


@pytest.mark.parametrize("M,n_exp,d,ff,n_act", [(100, 8, 256, 256, 8),     # every expert in every row: 13 chunks each
                                                (40, 16, 512, 256, 4), (17, 64, 1024, 512, 2),
                                                (33, 200, 256, 256, 6),
                                                (12, 8, 3072, 512, 2)])   # d of 12 blocks: the router's general form
def test_moe_many_rows_small_shapes(dev, M, n_exp, d, ff, n_act):
    check(M, n_exp, d, ff, n_act, seed=620 + M + n_exp, dev=dev)


@pytest.mark.parametrize("M,n_exp,d,ff,n_act", [(8, 16, 512, 4096, 4),    # union-slot down (ff of 16 super-blocks)
                                                (8, 200, 256, 256, 6),     # fused down, two row groups
                                                (6, 16, 512, 4096, 8)])    # 48 pairs, union-slot down
def test_moe_eight_rows_small_shapes(dev, M, n_exp, d, ff, n_act):
    # 6 and 8 rows at small shapes: the fused down projection in row groups where it fits LDS,
    # else the union-slot down kernel and the separate combine
    check(M, n_exp, d, ff, n_act, seed=780 + n_exp + M, dev=dev)


def test_moe_few_rows_large_ff(dev):
    # 3 rows x 8 experts with ff = 4096: the fused down projection does not fit LDS, so the
    # union-slot down kernel and the separate combine run
    check(3, 16, 512, 4096, 8, seed=790, dev=dev)


@pytest.mark.parametrize("M", [3, 8, 16])
def test_moe_largest_hidden_and_ff(dev, M):
    # d = ff = 4096, the largest the kernels take: 16 super-blocks per row (router rows of 16
    # blocks per lane, 128 KiB of staged activations per matrix-core block)
    check(M, 4, 4096, 4096, 2, seed=760, dev=dev)


def test_moe_many_rows_residual(dev):
    check(33, 128, 2048, 768, 8, seed=530, dev=dev, residual=True)


def test_moe_many_rows_equal_single_rows(dev):
    L = layer(128, 2048, 768, 500, dev)
    hn = synth.normal_f32(840, (24, 2048))
    out, sel, sw = gpu_moe(hn, L, 8, dev)
    for m in (0, 7, 8, 15, 23):
        o1, s1, w1 = gpu_moe(hn[m:m + 1], L, 8, dev)
        assert np.array_equal(sel[m], s1[0])
        assert np.array_equal(out[m].view(np.uint32), o1[0].view(np.uint32)), "row %d differs" % m


def test_moe_rejects_too_many_rows(dev):
    L = layer(16, 512, 256, 700, dev)
    import torch
    hn = torch.zeros((513, 512), device=dev)
    out = torch.zeros((513, 512), device=dev)
    with pytest.raises(x100hip.X100Error):
        x100hip.moe_layer(513, 512, 256, 16, 4, hn.data_ptr(), L[5].data_ptr(), L[4][0].data_ptr(),
                          L[4][1].data_ptr(), L[4][2].data_ptr(), out.data_ptr(), False, None, None)
