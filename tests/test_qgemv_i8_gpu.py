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


def test_requant_scale_truncation_edges(dev):
    """The device's fp16 truncation (the reference's f32_to_f16) over every branch: Q8_0 blocks
    whose requantized step amax/127 is fp16-normal with dropped bits, fp16-subnormal, below the
    smallest subnormal (the 1e-6 floor of an all-zero block) and at the top of the fp16 range;
    checked against the oracle and against the truncation's closed form."""
    import refseq
    rng = np.random.default_rng(5)
    nb = 64 * 8
    W = np.zeros((64, 8), synth.DT_Q8_0)
    q = rng.integers(-120, 121, size=(64, 8, 32)).astype(np.int8)
    q[:, 4:, 0] = 127                                  # amax = 127 * d: the step is d itself
    W["qs"] = q                                        # elsewhere the step drops bits
    # input scales (fp16 bits): normal, subnormal, tiny subnormal, large
    d_in = np.concatenate([rng.integers(0x0400, 0x7800, size=nb // 4),      # normal
                           rng.integers(0x0001, 0x0400, size=nb // 4),      # subnormal
                           rng.integers(0x0001, 0x0008, size=nb // 4),      # a few subnormal steps
                           rng.integers(0x7800, 0x7BFF, size=nb // 4)]).astype(np.uint16)
    W["d"] = d_in.reshape(64, 8)
    W["qs"][5] = 0                                     # all-zero rows: amax floored at 1e-6
    W["d"][6] = 0x7BFF                                 # 65504 * 127 / 127
    packed = gpu_pack(synth.Q8_0, W, 256, dev)
    ref = ol.requant_q8_0(synth.Q8_0, W).reshape(-1)
    d = packed[:nb * 2].view(np.uint16)
    assert np.array_equal(d, ref["d"]), "scales differ from the oracle"
    assert np.array_equal(d, refseq.requant_q8_0(synth.Q8_0, W)[0].reshape(-1)), "scales differ from the truncation"
    assert (d[5 * 8:6 * 8] == 0).all()                 # 1e-6 / 127 truncates to zero
    qs_off = (nb * 2 + 255) // 256 * 256
    assert np.array_equal(packed[qs_off:qs_off + nb * 32].view(np.int8).reshape(nb, 32), ref["qs"])
    # a step of 2^16 or more (only reachable from a K-quant source) gives infinity
    W6 = synth.quant_weight(synth.Q6_K, 1, 256, seed=3)
    W6["d"] = 0x7BFF
    W6["scales"] = 127
    W6["ql"], W6["qh"] = 0xFF, 0xFF                    # q = 63 - 32 = 31 everywhere
    d6 = gpu_pack(synth.Q6_K, W6, 256, dev)[:16].view(np.uint16)
    assert np.array_equal(d6, ol.requant_q8_0(synth.Q6_K, W6)["d"].reshape(-1))
    assert (d6 == 0x7C00).all()


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
