"""Caller-scoped scratch of the MoE block and the decode layer (the _ws entry points) and the
per-stream workspaces of the convenience entry points: any initial scratch contents, two layers
running concurrently on two streams, a HIP graph captured at a shape larger than any earlier call
and replayed with other work in between, and argument errors that leave every buffer untouched.
Results are compared with the oracle bit for bit."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip
from test_moe_gpu import layer

pytestmark = pytest.mark.gpu

D, FF, NE, NA = 2048, 768, 128, 8


def dev_ptrs(L):
    Wg, Wu, Wd, R, dW, dR = L
    return dR.data_ptr(), dW[0].data_ptr(), dW[1].data_ptr(), dW[2].data_ptr()


def oracle_out(L, hn):
    Wg, Wu, Wd, R = L[:4]
    return ol.moe_layer(hn, R, Wg, Wu, Wd, NA)


def same_bits(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_moe_workspace_size_query(dev):
    assert x100hip.moe_workspace_bytes(1, D, FF, NE, NA) > 0
    assert x100hip.moe_workspace_bytes(16, D, FF, NE, NA) > x100hip.moe_workspace_bytes(4, D, FF, NE, NA)
    assert x100hip.moe_workspace_bytes(1, D, FF, NE, NA) % 256 == 0
    for bad in ((0, D, FF, NE, NA), (513, D, FF, NE, NA), (1, 100, FF, NE, NA), (1, D, FF, 4, 8),
                (1, D, FF, NE, 9), (1, 8192, FF, NE, NA)):
        assert x100hip.moe_workspace_bytes(*bad) == 0, bad


@pytest.mark.parametrize("M", [1, 4, 16])
def test_moe_ws_any_initial_contents(dev, M):
    """Scratch filled with 0xff bytes, then with a float pattern: same bits as the oracle."""
    import torch
    L = layer(NE, D, FF, 500, dev)
    dR, dg, du, dd = dev_ptrs(L)
    hn = synth.normal_f32(900 + M, (M, D))
    ref, rsel, rsw = oracle_out(L, hn)
    nb = x100hip.moe_workspace_bytes(M, D, FF, NE, NA)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    dh = torch.from_numpy(hn).to(dev)
    s = torch.cuda.current_stream().cuda_stream
    for fill in (0xFF, 0x7F):
        ws.fill_(fill)
        out = torch.full((M, D), float("nan"), device=dev)
        sel = torch.full((M, NA), -1, dtype=torch.int32, device=dev)
        sw = torch.zeros((M, NA), device=dev)
        x100hip.moe_layer_ws(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, out.data_ptr(), False, sel.data_ptr(),
                             sw.data_ptr(), ws.data_ptr(), nb, s)
        torch.cuda.synchronize()
        assert same_bits(out.cpu().numpy(), ref)
        assert np.array_equal(sel.cpu().numpy(), rsel) and same_bits(sw.cpu().numpy(), rsw)


def test_moe_ws_rejects_small_or_misaligned_scratch(dev):
    import torch
    L = layer(NE, D, FF, 500, dev)
    dR, dg, du, dd = dev_ptrs(L)
    nb = x100hip.moe_workspace_bytes(2, D, FF, NE, NA)
    ws = torch.empty(nb + 256, dtype=torch.uint8, device=dev)
    hn = torch.zeros((2, D), device=dev)
    out = torch.full((2, D), 3.0, device=dev)
    for ptr, size in ((ws.data_ptr(), nb - 256), (ws.data_ptr() + 16, nb), (0, nb)):
        with pytest.raises(x100hip.X100Error):
            x100hip.moe_layer_ws(2, D, FF, NE, NA, hn.data_ptr(), dR, dg, du, dd, out.data_ptr(), False, None, None,
                                 ptr, size)
    torch.cuda.synchronize()
    assert (out == 3.0).all()   # nothing was enqueued


def test_moe_two_streams_concurrent(dev):
    """Two layers (4 rows and 1 row, different inputs) on two streams, each with its own scratch,
    enqueued alternately with no synchronisation between them; then the convenience entry point
    on the same two streams (one library workspace per stream)."""
    import torch
    L = layer(NE, D, FF, 500, dev)
    dR, dg, du, dd = dev_ptrs(L)
    cases = [(4, synth.normal_f32(950, (4, D))), (1, synth.normal_f32(951, (1, D)))]
    refs = [oracle_out(L, hn)[0] for _, hn in cases]
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    bufs = []
    for (M, hn) in cases:
        nb = x100hip.moe_workspace_bytes(M, D, FF, NE, NA)
        bufs.append((torch.from_numpy(hn).to(dev), torch.empty(nb, dtype=torch.uint8, device=dev).fill_(0xFF), nb,
                     [torch.full((M, D), float("nan"), device=dev) for _ in range(4)]))
    torch.cuda.synchronize()
    for it in range(4):
        for k, ((M, _), (dh, ws, nb, outs), st) in enumerate(zip(cases, bufs, streams)):
            x100hip.moe_layer_ws(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, outs[it].data_ptr(), False, None,
                                 None, ws.data_ptr(), nb, st.cuda_stream)
    torch.cuda.synchronize()
    for k in range(2):
        for it in range(4):
            assert same_bits(bufs[k][3][it].cpu().numpy(), refs[k]), "stream %d call %d" % (k, it)
    # convenience form: a workspace per stream
    for it in range(3):
        for k, ((M, _), (dh, _, _, outs), st) in enumerate(zip(cases, bufs, streams)):
            outs[it].fill_(float("nan"))
    torch.cuda.synchronize()
    for it in range(3):
        for k, ((M, _), (dh, _, _, outs), st) in enumerate(zip(cases, bufs, streams)):
            x100hip.moe_layer(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, outs[it].data_ptr(), False, None, None,
                              st.cuda_stream)
    torch.cuda.synchronize()
    for k in range(2):
        for it in range(3):
            assert same_bits(bufs[k][3][it].cpu().numpy(), refs[k]), "convenience stream %d call %d" % (k, it)


def test_moe_per_thread_stream_two_threads(dev):
    """hipStreamPerThread is one handle for a different stream in each host thread: two threads
    calling the convenience entry point with it at once (4 rows and 1 row) each get a workspace of
    their own, and every output equals the oracle's."""
    import threading
    import torch
    HIP_STREAM_PER_THREAD = 2   # (hipStream_t)2
    L = layer(NE, D, FF, 500, dev)
    dR, dg, du, dd = dev_ptrs(L)
    cases = [(4, synth.normal_f32(970, (4, D))), (1, synth.normal_f32(971, (1, D)))]
    refs = [oracle_out(L, hn)[0] for _, hn in cases]
    reps = 6
    bufs = [(torch.from_numpy(hn).to(dev), [torch.full((M, D), float("nan"), device=dev) for _ in range(reps)])
            for M, hn in cases]
    torch.cuda.synchronize()
    errs = []

    def run(k):
        try:
            M = cases[k][0]
            dh, outs = bufs[k]
            for it in range(reps):
                x100hip.moe_layer(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, outs[it].data_ptr(), False, None,
                                  None, HIP_STREAM_PER_THREAD)
            torch.cuda.synchronize()
        except Exception as e:   # collected and re-raised in the main thread
            errs.append(e)

    ts = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert not errs, errs
    for k in range(2):
        for it in range(reps):
            assert same_bits(bufs[k][1][it].cpu().numpy(), refs[k]), "thread %d call %d" % (k, it)


def test_moe_graph_captured_at_a_larger_shape(dev):
    """A graph holding moe_layer_hip_ws at 16 rows, after eager calls at 2 rows only: three
    replays, with eager layers and synchronisations between them, each bit-identical to the
    oracle.  The convenience entry point refuses to grow its workspace during a capture."""
    import torch
    L = layer(NE, D, FF, 500, dev)
    dR, dg, du, dd = dev_ptrs(L)
    s0 = torch.cuda.current_stream().cuda_stream
    small = torch.from_numpy(synth.normal_f32(960, (2, D))).to(dev)
    small_out = torch.empty((2, D), device=dev)
    x100hip.moe_layer(2, D, FF, NE, NA, small.data_ptr(), dR, dg, du, dd, small_out.data_ptr(), False, None, None,
                      s0)
    M = 16
    hn = synth.normal_f32(961, (M, D))
    ref = oracle_out(L, hn)[0]
    dh = torch.from_numpy(hn).to(dev)
    nb = x100hip.moe_workspace_bytes(M, D, FF, NE, NA)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev).fill_(0xFF)
    out = torch.full((M, D), float("nan"), device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    refused = False
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream().cuda_stream
        x100hip.moe_layer_ws(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, out.data_ptr(), False, None, None,
                             ws.data_ptr(), nb, cs)
        try:   # the capture stream has no library workspace yet: growing one is refused
            x100hip.moe_layer(M, D, FF, NE, NA, dh.data_ptr(), dR, dg, du, dd, out.data_ptr(), False, None, None,
                              cs)
        except x100hip.X100Error as e:
            refused = e.code == x100hip.X100_EINVAL
    assert refused
    small_ref = oracle_out(L, synth.normal_f32(960, (2, D)))[0]
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert same_bits(out.cpu().numpy(), ref), "replay %d" % rep
        # eager work between replays, on the library's workspace of the default stream
        x100hip.moe_layer(2, D, FF, NE, NA, small.data_ptr(), dR, dg, du, dd, small_out.data_ptr(), False, None,
                          None, s0)
        torch.cuda.synchronize()
        assert same_bits(small_out.cpu().numpy(), small_ref)


# ------------------------------------------------------------------------------------------------
# decode layer
# ------------------------------------------------------------------------------------------------
def qwen_layer(dev):
    from test_decode_gpu import GpuLayer
    from test_decode_oracle import make_cfg
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    cfg = make_cfg(types, d=2048, n_head=32, n_head_kv=4, ff=768, n_exp=128, n_act=8, ctx=512)
    L = synth.decode_layer_weights(2048, 32, 4, 128, 768, 128, types, seed=140)
    return cfg, L, GpuLayer(cfg, L, types, dev)


def test_decode_layer_ws_equals_oracle_and_convenience(dev):
    import torch
    from test_decode_oracle import caches
    cfg, L, gl = qwen_layer(dev)
    nb = x100hip.decode_workspace_bytes(gl.gcfg)
    assert nb > 0 and nb % 256 == 0
    ws = torch.empty(nb, dtype=torch.uint8, device=dev).fill_(0xFF)
    s = torch.cuda.current_stream().cuda_stream
    pos = 300
    kc, vc = caches(cfg, pos, 620)
    h = synth.normal_f32(621, (cfg.d,))
    rh, rk, rv = h.copy(), kc.copy(), vc.copy()
    rsel, rsw = ol.decode_layer(cfg, L, rk, rv, pos, rh)
    for use_ws in (True, False):
        gl.set_cache(kc, vc)
        dh = torch.from_numpy(h.copy()).to(dev)
        sel = torch.full((8,), -1, dtype=torch.int32, device=dev)
        sw = torch.zeros(8, device=dev)
        if use_ws:
            x100hip.decode_layer_ws(gl.gcfg, gl.w, pos, dh.data_ptr(), sel.data_ptr(), sw.data_ptr(), ws.data_ptr(),
                                    nb, s)
        else:
            x100hip.decode_layer(gl.gcfg, gl.w, pos, dh.data_ptr(), sel.data_ptr(), sw.data_ptr(), s)
        torch.cuda.synchronize()
        assert same_bits(dh.cpu().numpy(), rh) and np.array_equal(sel.cpu().numpy(), rsel)
        assert same_bits(sw.cpu().numpy(), rsw)
        assert same_bits(gl.kc.cpu().numpy()[:, pos], rk[:, pos])
    # attention half alone on caller scratch (its share is smaller than the whole layer's)
    gl.set_cache(kc, vc)
    dh = torch.from_numpy(h.copy()).to(dev)
    x100hip.attn_decode_ws(gl.gcfg, gl.w, pos, dh.data_ptr(), ws.data_ptr(), nb, s)
    torch.cuda.synchronize()
    rh2, rk2, rv2 = h.copy(), kc.copy(), vc.copy()
    ol.attn_decode(cfg, L, rk2, rv2, pos, rh2)
    assert same_bits(dh.cpu().numpy(), rh2)
    with pytest.raises(x100hip.X100Error):
        x100hip.decode_layer_ws(gl.gcfg, gl.w, pos, dh.data_ptr(), None, None, ws.data_ptr(), nb - 256, s)


def test_decode_layer_argument_error_leaves_state_untouched(dev):
    """A misaligned MoE pointer is caught before the attention half runs: h and the KV cache are
    unchanged (a retry does not apply the attention residual twice)."""
    import torch
    from test_decode_oracle import caches
    cfg, L, gl = qwen_layer(dev)
    pos = 10
    kc, vc = caches(cfg, pos, 630)
    gl.set_cache(kc, vc)
    h = synth.normal_f32(631, (cfg.d,))
    dh = torch.from_numpy(h.copy()).to(dev)
    w_bad = x100hip.LayerWeights(*[getattr(gl.w, n) for n, _ in x100hip.LayerWeights._fields_])
    w_bad.router = gl.w.router + 4
    with pytest.raises(x100hip.X100Error):
        x100hip.decode_layer(gl.gcfg, w_bad, pos, dh.data_ptr())
    c_bad = x100hip.LayerCfg(*[getattr(gl.gcfg, n) for n, _ in x100hip.LayerCfg._fields_])
    c_bad.n_act = 9
    with pytest.raises(x100hip.X100Error):
        x100hip.decode_layer(c_bad, gl.w, pos, dh.data_ptr())
    torch.cuda.synchronize()
    assert same_bits(dh.cpu().numpy(), h)
    assert np.array_equal(gl.kc.cpu().numpy(), kc) and np.array_equal(gl.vc.cpu().numpy(), vc)
