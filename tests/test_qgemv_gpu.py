"""Q4_0 / Q4_K / Q3_K dequant-GEMV on the GPU against the oracle: bit for bit (the oracle combines
the per-block dots in the kernels' order), and within rel 1e-3 / abs 1e-4 in fp32 besides."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


def gpu_qgemv(qtype, W, x, dev):
    import torch
    N = W.shape[0]
    M, K = x.shape
    s = torch.cuda.current_stream().cuda_stream
    raw = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
    packed = torch.empty(x100hip.packed_bytes(qtype, N, K), dtype=torch.uint8, device=dev)
    x100hip.pack(qtype, N, K, raw.data_ptr(), packed.data_ptr(), s)
    dx = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
    dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    x100hip.qgemv(qtype, M, N, K, packed.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
    torch.cuda.synchronize()
    return dy.cpu().numpy()


def check(qtype, N, K, M, seed, dev, exact=None):
    W = synth.quant_weight(qtype, N, K, seed)
    x = synth.normal_f32(seed + 1, (M, K))
    got = gpu_qgemv(qtype, W, x, dev)
    ref = ol.qgemv(qtype, W, x)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), "qtype %d N=%d K=%d M=%d: %d outside tolerance, max err %g" % (
        qtype, N, K, M, int(bad.sum()), float(err.max()))
    if exact is None:
        exact = True
    if exact:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "not bit-identical"


def check_reference_order(qtype, N, K, M, seed, dev):
    """The benchmark configurations: bit-identical to the oracle, and within rel 1e-3 / abs 1e-4
    of the reference's own checking arithmetic (tests/refseq.py) on every element."""
    import refseq
    check(qtype, N, K, M, seed, dev)
    W = synth.quant_weight(qtype, N, K, seed)
    x = synth.normal_f32(seed + 1, (M, K))
    got = gpu_qgemv(qtype, W, x, dev)
    ref = refseq.gemv(qtype, W, x)
    bad = np.abs(got - ref) > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), "%d elements outside tolerance of the reference order" % int(bad.sum())


@pytest.mark.parametrize("M", [1, 4])
def test_q4_0_4096(dev, M):
    check_reference_order(synth.Q4_0, 4096, 4096, M, seed=300 + M, dev=dev)


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q3_K])
@pytest.mark.parametrize("M", [1, 4])
def test_kquant_6144x2048(dev, qtype, M):
    check_reference_order(qtype, 6144, 2048, M, seed=400 + M + qtype, dev=dev)


@pytest.mark.parametrize("qtype,N,K,M", [
    (synth.Q4_0, 1, 32, 1), (synth.Q4_0, 7, 96, 2), (synth.Q4_0, 300, 2048, 3), (synth.Q4_0, 64, 8192, 8),
    (synth.Q4_0, 130, 1024, 6),
    (synth.Q4_0, 33, 16384, 1), (synth.Q4_K, 1, 256, 1), (synth.Q4_K, 5, 768, 2), (synth.Q4_K, 2048, 768, 8),
    (synth.Q4_K, 100, 4096, 3), (synth.Q4_K, 9, 8192, 1), (synth.Q3_K, 1, 256, 1), (synth.Q3_K, 13, 768, 5),
    (synth.Q3_K, 700, 4096, 8), (synth.Q3_K, 3, 16384, 2),
    # the several-row kernels (2 to 8 token rows): ragged row tiles, odd super-block counts
    (synth.Q4_K, 17, 2560, 7), (synth.Q3_K, 31, 1280, 6), (synth.Q4_K, 6144, 2048, 2),
    (synth.Q3_K, 6144, 2048, 8), (synth.Q4_K, 4100, 4096, 5), (synth.Q3_K, 16, 256, 4),
    # one token row with 3 or 16 super-blocks per row (the four-lane kernels, not the row-major one)
    (synth.Q3_K, 40, 768, 1), (synth.Q4_K, 300, 4096, 1), (synth.Q3_K, 257, 4096, 1)])
def test_qgemv_shapes(dev, qtype, N, K, M):
    check(qtype, N, K, M, seed=N + K + M, dev=dev)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q4_K, synth.Q3_K])
def test_qgemv_zero_activation(dev, qtype):
    W = synth.quant_weight(qtype, 64, 512, seed=9)
    y = gpu_qgemv(qtype, W, np.zeros((2, 512), np.float32), dev)
    assert not y.any()


def test_qgemv_rejects_bad_shapes(dev):
    with pytest.raises(x100hip.X100Error):
        x100hip.qgemv(synth.Q4_K, 1, 16, 100, 1 << 20, 1 << 20, 1 << 20)
    with pytest.raises(x100hip.X100Error):
        x100hip.qgemv(synth.Q4_0, 9, 16, 64, 1 << 20, 1 << 20, 1 << 20)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q4_K, synth.Q3_K])
@pytest.mark.parametrize("M", [4, 8])
def test_qgemv_batched_rows_equal_single_rows(dev, qtype, M):
    # the multi-row block shapes (more waves, one row per wave for Q4_0) compute each row exactly
    # as the one-row kernels do: per-row quantization, same per-block order
    N, K = 1024, 2048
    W = synth.quant_weight(qtype, N, K, seed=900 + qtype)
    x = synth.normal_f32(901 + M, (M, K))
    y = gpu_qgemv(qtype, W, x, dev)
    for m in range(M):
        y1 = gpu_qgemv(qtype, W, x[m:m + 1], dev)
        assert np.array_equal(y[m].view(np.uint32), y1[0].view(np.uint32)), "row %d differs" % m


def _fbits(f):
    import struct
    return struct.unpack("<I", struct.pack("<f", f))[0]


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def test_quantizer_division_free_arithmetic_is_exact(dev):
    # The activation quantizers compute amax / 127.0f, 1.0f / d and d's fp16 truncation without
    # IEEE division.  Exhaustively on this GPU: 1/d over every positive d up to FLT_MAX / 127
    # (subnormal d included: the Q8_K quantizers have no amax floor), amax / 127 over every
    # positive amax, and the fp16 truncation over every positive float; zero mismatches against
    # the correctly rounded quotients and the reference's conversion (the check kernel runs
    # the quantizers' own device functions).
    import torch
    fmax = 0x7f7fffff
    d_hi = _fbits(np.float32(3.4028234663852886e38 / 127.0))
    cnt = torch.zeros(3, dtype=torch.int64, device=dev)
    x100hip.check_quant_div(1, d_hi, cnt.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert int(cnt[0]) == 0, "1/d mismatches over the d range: %d" % int(cnt[0])
    cnt.zero_()
    x100hip.check_quant_div(1, fmax, cnt.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert int(cnt[1]) == 0, "div127_rn mismatches: %d" % int(cnt[1])
    assert int(cnt[2]) == 0, "f16_trunc_pos mismatches: %d" % int(cnt[2])
