"""moe_layer_hip_noalloc: the MoE block with its scratch in the library's static per-GPU array.
Two calls in a row (16 token rows, then 2) must give exactly what moe_layer_hip gives for the
same inputs, and the oracle's bits, without allocating device memory; a shape needing more
scratch than the array holds is refused with X100_ESCRATCH and nothing enqueued."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip
from test_moe_gpu import layer

pytestmark = pytest.mark.gpu

D, FF, NE, NA = 2048, 768, 128, 8


def call(fn, L, hn, dev, stream):
    import torch
    Wg, Wu, Wd, R, dW, dR = L
    M = hn.shape[0]
    dh = torch.from_numpy(hn).to(dev)
    out = torch.full((M, D), float("nan"), device=dev)
    sel = torch.full((M, NA), -1, dtype=torch.int32, device=dev)
    sw = torch.zeros((M, NA), device=dev)
    torch.cuda.synchronize()
    return dh, out, sel, sw, lambda: fn(M, D, FF, NE, NA, dh.data_ptr(), dR.data_ptr(), dW[0].data_ptr(),
                                        dW[1].data_ptr(), dW[2].data_ptr(), out.data_ptr(), False, sel.data_ptr(),
                                        sw.data_ptr(), stream)


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def test_noalloc_matches_moe_layer_hip(dev):
    import torch
    L = layer(NE, D, FF, 500, dev)
    s = torch.cuda.current_stream().cuda_stream
    print("noalloc: 16 rows, then 2 rows, then the same through moe_layer_hip", flush=True)
    inputs = [synth.normal_f32(970, (16, D)), synth.normal_f32(971, (2, D))]
    # warm-up call (loads the library's code object on a fresh process), then the measured calls
    w = call(x100hip.moe_layer_noalloc, L, synth.normal_f32(972, (1, D)), dev, s)
    w[4]()
    torch.cuda.synchronize()
    prepared = [call(x100hip.moe_layer_noalloc, L, hn, dev, s) for hn in inputs]
    free0 = torch.cuda.mem_get_info()[0]
    for p in prepared:
        p[4]()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 >= free0, "device memory was allocated (%d bytes)" % (free0 - free1)
    for hn, p in zip(inputs, prepared):
        _, out, sel, sw, _ = p
        q = call(x100hip.moe_layer, L, hn, dev, s)
        q[4]()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), bits(q[1])), "M=%d: differs from moe_layer_hip" % hn.shape[0]
        assert np.array_equal(sel.cpu().numpy(), q[2].cpu().numpy()) and np.array_equal(bits(sw), bits(q[3]))
        Wg, Wu, Wd, R = L[:4]
        ref, rsel, rsw = ol.moe_layer(hn, R, Wg, Wu, Wd, NA)
        assert np.array_equal(bits(out), ref.view(np.uint32)), "M=%d: differs from the oracle" % hn.shape[0]


def test_noalloc_refuses_shapes_beyond_the_array(dev):
    import torch
    L = layer(NE, D, FF, 500, dev)
    M = 128
    assert x100hip.moe_workspace_bytes(M, D, FF, NE, NA) > x100hip.MOE_NOALLOC_MAX_BYTES
    assert x100hip.moe_workspace_bytes(64, D, FF, NE, NA) <= x100hip.MOE_NOALLOC_MAX_BYTES
    p = call(x100hip.moe_layer_noalloc, L, synth.normal_f32(973, (M, D)), dev,
             torch.cuda.current_stream().cuda_stream)
    with pytest.raises(x100hip.X100Error) as e:
        p[4]()
    assert e.value.code == x100hip.X100_ESCRATCH
    torch.cuda.synchronize()
    assert torch.isnan(p[1]).all()   # nothing was enqueued
