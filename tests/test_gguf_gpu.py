"""Tensors of a GGUF file go from the mapping to the GPU kernels as they are: the MoE layer runs on
the expert tensors uploaded by x100_gguf_upload, the GEMVs on rows packed by x100_gguf_pack_rows,
and both match the oracle on the same blocks (MoE bit for bit, GEMV to rel 1e-3 / abs 1e-4)."""
import numpy as np
import pytest

import gguf
import oracle_lib as ol
import synth
import x100hip
from test_gguf import qwen_like
from test_qgemv_gpu import ATOL, RTOL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "m.gguf")
    kv, ten = qwen_like()
    gguf.write(path, kv, ten)
    g = gguf.GGUF(path)
    yield g
    g.close()


def blocks(t, qt):
    """The tensor's bytes as N rows of GGUF blocks (numpy structured), N = elements / dims[0]."""
    K = t.dims[0]
    dt = {synth.Q4_0: synth.DT_Q4_0, synth.Q8_0: synth.DT_Q8_0, synth.Q3_K: synth.DT_Q3_K,
          synth.Q4_K: synth.DT_Q4_K, synth.Q5_K: synth.DT_Q5_K, synth.Q6_K: synth.DT_Q6_K}[qt]
    return t.array().view(dt).reshape(-1, K // synth.BLOCK_ELEMS[qt]).copy()


def test_moe_layer_from_gguf(model, dev):
    import torch
    g = model
    p = g.qwen3moe()
    d, ff, n_exp, n_act = p["embd"], p["moe_ffn"], p["n_exp"], p["n_act"]
    s = torch.cuda.current_stream().cuda_stream
    dev_t = {}
    for name in ("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight", "blk.0.ffn_down_exps.weight",
                 "blk.0.ffn_gate_inp.weight"):
        t = g.find(name)
        buf = torch.empty(t.n_bytes, dtype=torch.uint8, device=dev)
        g.upload(t, buf.data_ptr(), s)
        dev_t[name] = (t, buf)
    tg, tu, td, tr = (dev_t[n][0] for n in ("blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                                            "blk.0.ffn_down_exps.weight", "blk.0.ffn_gate_inp.weight"))
    assert tg.shape == (d, ff, n_exp) and td.shape == (ff, d, n_exp) and tr.shape == (d, n_exp)
    Wg = blocks(tg, synth.Q4_K).reshape(n_exp, ff, d // 256)
    Wu = blocks(tu, synth.Q4_K).reshape(n_exp, ff, d // 256)
    Wd = blocks(td, synth.Q4_K).reshape(n_exp, d, ff // 256)
    R = tr.array().view(np.float32).reshape(n_exp, d).copy()
    for M in (1, 4):
        hn = synth.normal_f32(700 + M, (M, d))
        dh = torch.from_numpy(hn).to(dev)
        out = torch.full((M, d), float("nan"), device=dev)
        sel = torch.full((M, n_act), -1, dtype=torch.int32, device=dev)
        sw = torch.zeros((M, n_act), dtype=torch.float32, device=dev)
        x100hip.moe_layer(M, d, ff, n_exp, n_act, dh.data_ptr(), dev_t["blk.0.ffn_gate_inp.weight"][1].data_ptr(),
                          dev_t["blk.0.ffn_gate_exps.weight"][1].data_ptr(),
                          dev_t["blk.0.ffn_up_exps.weight"][1].data_ptr(),
                          dev_t["blk.0.ffn_down_exps.weight"][1].data_ptr(), out.data_ptr(), False, sel.data_ptr(),
                          sw.data_ptr(), s)
        torch.cuda.synchronize()
        ref, rsel, rsw = ol.moe_layer(hn, R, Wg, Wu, Wd, n_act)
        assert np.array_equal(sel.cpu().numpy(), rsel) and np.array_equal(sw.cpu().numpy(), rsw)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name,qt", [("output.weight", synth.Q6_K), ("blk.0.attn_k.weight", synth.Q8_0),
                                     ("blk.0.attn_v.weight", synth.Q4_0), ("blk.0.attn_q.weight", synth.Q3_K),
                                     ("blk.0.attn_output.weight", synth.Q5_K)])
def test_gemv_from_gguf_rows(model, dev, name, qt):
    import torch
    g = model
    t = g.find(name)
    assert t.type == qt
    K, N = t.dims[0], t.n_elems // t.dims[0]
    s = torch.cuda.current_stream().cuda_stream
    W = blocks(t, qt)
    x = synth.normal_f32(800 + qt, (3, K))
    dx = torch.from_numpy(x).to(dev)
    ref = ol.qgemv(qt, W, x)
    # the whole tensor, and a row range of it (rows r0 .. r0 + n of the same GEMV)
    for r0, n in ((0, N), (N // 3, N // 2)):
        pk = torch.empty(x100hip.packed_bytes(qt, n, K), dtype=torch.uint8, device=dev)
        g.pack_rows(t, r0, n, pk.data_ptr(), s)
        dy = torch.full((3, n), float("nan"), device=dev)
        x100hip.qgemv(qt, 3, n, K, pk.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        got = dy.cpu().numpy()
        err = np.abs(got - ref[:, r0:r0 + n])
        assert np.all(err <= ATOL + RTOL * np.abs(ref[:, r0:r0 + n])), (name, r0, float(err.max()))


def test_expert_slice_from_gguf(model, dev):
    # one expert's gate matrix out of the 3-D tensor: rows e*ff .. (e+1)*ff
    import torch
    g = model
    t = g.find("blk.0.ffn_gate_exps.weight")
    d, ff, n_exp = t.shape
    s = torch.cuda.current_stream().cuda_stream
    W = blocks(t, synth.Q4_K).reshape(n_exp, ff, d // 256)
    x = synth.normal_f32(901, (1, d))
    dx = torch.from_numpy(x).to(dev)
    for e in (0, n_exp - 1):
        pk = torch.empty(x100hip.packed_bytes(synth.Q4_K, ff, d), dtype=torch.uint8, device=dev)
        g.pack_rows(t, e * ff, ff, pk.data_ptr(), s)
        dy = torch.empty((1, ff), device=dev)
        x100hip.qgemv(synth.Q4_K, 1, ff, d, pk.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        ref = ol.qgemv(synth.Q4_K, W[e], x)
        assert np.array_equal(dy.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_pack_rows_rejects_bad_ranges(model, dev):
    import torch
    g = model
    t = g.find("output.weight")
    N = t.n_elems // t.dims[0]
    buf = torch.empty(x100hip.packed_bytes(synth.Q6_K, 8, t.dims[0]), dtype=torch.uint8, device=dev)
    for r0, n in ((N - 4, 8), (N + 1, 1), (0, 0)):
        with pytest.raises(x100hip.X100Error):
            g.pack_rows(t, r0, n, buf.data_ptr())
    with pytest.raises(x100hip.X100Error):
        g.pack_rows(g.find("blk.0.attn_norm.weight"), 0, 1, buf.data_ptr())   # F32: not a qgemv type
