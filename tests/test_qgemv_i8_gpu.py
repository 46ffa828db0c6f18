"""Int8 path of the quantized GEMV on the GPU: Q8_0 / Q5_K / Q6_K weights requantized to Q8_0 at
load (lin_new_i8, qwen_moe_q3k.c:872-886) and multiplied with pack_A_i8 activations
(run_i8_m1, :428-510).  The requantized weight and the GEMV output are compared with the oracle's
bit for bit (the oracle combines the blocks in the kernel's lane order), and within
rel 1e-3 / abs 1e-4 besides."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip
from test_qgemv_gpu import RTOL, ATOL, gpu_qgemv

pytestmark = pytest.mark.gpu
I8_TYPES = [synth.Q8_0, synth.Q5_K, synth.Q6_K]


def gpu_pack(qtype, W, K, dev):
    import torch
    N = W.shape[0]
    raw = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
    packed = torch.full((x100hip.packed_bytes(qtype, N, K),), 0xAB, dtype=torch.uint8, device=dev)
    x100hip.pack(qtype, N, K, raw.data_ptr(), packed.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return packed.cpu().numpy()


def check(qtype, N, K, M, seed, dev):
    W = synth.quant_weight(qtype, N, K, seed)
    x = synth.normal_f32(seed + 1, (M, K))
    got = gpu_qgemv(qtype, W, x, dev)
    ref = ol.qgemv(qtype, W, x)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), "qtype %d N=%d K=%d M=%d: %d outside tolerance, max err %g" % (
        qtype, N, K, M, int(bad.sum()), float(err.max()))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "not bit-identical"


@pytest.mark.parametrize("qtype,N,K", [(synth.Q8_0, 37, 512), (synth.Q5_K, 300, 2048), (synth.Q6_K, 129, 1024),
                                       (synth.Q8_0, 1, 32), (synth.Q6_K, 1, 256)])
def test_requant_matches_oracle(dev, qtype, N, K):
    W = synth.quant_weight(qtype, N, K, seed=500 + qtype + N)
    packed = gpu_pack(qtype, W, K, dev)
    ref = ol.requant_q8_0(qtype, W).reshape(-1)
    ng = N * (K // 32)
    qs_off = (ng * 2 + 255) // 256 * 256
    d = packed[:ng * 2].view(np.uint16)
    qs = packed[qs_off:qs_off + ng * 32].view(np.int8).reshape(ng, 32)
    assert np.array_equal(d, ref["d"]), "scales differ"
    assert np.array_equal(qs, ref["qs"]), "values differ"


@pytest.mark.parametrize("qtype,N,K,M", [
    (synth.Q8_0, 512, 2048, 1),            # attn_k of Qwen3-30B-A3B
    (synth.Q5_K, 2048, 4096, 1),           # attn_output
    (synth.Q5_K, 2048, 4096, 4),
    (synth.Q6_K, 4096, 2048, 1),
    (synth.Q6_K, 4096, 2048, 8),
    (synth.Q8_0, 1, 32, 1), (synth.Q8_0, 7, 96, 2), (synth.Q6_K, 33, 256, 3), (synth.Q5_K, 5, 768, 8),
    (synth.Q8_0, 130, 16384, 1), (synth.Q6_K, 65, 8192, 5), (synth.Q8_0, 100, 4096, 6),
    (synth.Q6_K, 50000, 2048, 1),          # several row groups per block
    (synth.Q8_0, 40000, 1024, 4)])
def test_i8_qgemv_shapes(dev, qtype, N, K, M):
    check(qtype, N, K, M, seed=N + K + M + qtype, dev=dev)


def test_i8_qgemv_lm_head(dev):
    # output.weight of Qwen3-30B-A3B: vocab 151936 x hidden 2048, Q6_K in the mixed checkpoint
    check(synth.Q6_K, 151936, 2048, 1, seed=77, dev=dev)


@pytest.mark.parametrize("qtype", I8_TYPES)
@pytest.mark.parametrize("M", [4, 8])
def test_i8_batched_rows_equal_single_rows(dev, qtype, M):
    N, K = 1024, 2048
    W = synth.quant_weight(qtype, N, K, seed=910 + qtype)
    x = synth.normal_f32(911 + M, (M, K))
    y = gpu_qgemv(qtype, W, x, dev)
    for m in range(M):
        y1 = gpu_qgemv(qtype, W, x[m:m + 1], dev)
        assert np.array_equal(y[m].view(np.uint32), y1[0].view(np.uint32)), "row %d differs" % m


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_i8_zero_activation(dev, qtype):
    W = synth.quant_weight(qtype, 64, 512, seed=19)
    assert not gpu_qgemv(qtype, W, np.zeros((2, 512), np.float32), dev).any()


def test_i8_rejects_bad_shapes(dev):
    with pytest.raises(x100hip.X100Error):
        x100hip.qgemv(synth.Q6_K, 1, 16, 100, 1 << 20, 1 << 20, 1 << 20)   # K % 256
    with pytest.raises(x100hip.X100Error):
        x100hip.qgemv(synth.Q8_0, 9, 16, 64, 1 << 20, 1 << 20, 1 << 20)    # M > 8
    with pytest.raises(x100hip.X100Error):
        x100hip.qgemv(synth.Q8_0, 1, 16, 32768, 1 << 20, 1 << 20, 1 << 20)  # K / 32 > 512
