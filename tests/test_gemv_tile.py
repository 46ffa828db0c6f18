"""Integer tile GEMV (bench/q4_gemv.c contract): packers on the CPU, kernels on the GPU.

y[M][N] = W[N][K] . x[M][K]^T with int8 x, int4 or int8 W, int32 y: integer work, so the GPU
result must equal the oracle (ref_gemv, bench/q4_gemv.c:101-103) bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip


def q4_gemv_inputs(N, K, M, seed):
    """W in the int4 range [-7, 7] and x full int8 range (the distribution of bench/q4_gemv.c:117-118,
    drawn from the seeded splitmix64 stream)."""
    r = synth.rand_bytes(seed, N * K + M * K)
    W = (r[:N * K].astype(np.int32) % 15 - 7).astype(np.int8).reshape(N, K)
    x = r[N * K:].view(np.int8).reshape(M, K).copy()
    return W, x


def unpack_int4(Wq, N, K):
    """Independent reading of the int4 layout: byte 16n+k of tile (nb, kp) -> W[8nb+n][32kp+k]
    (low nibble) and W[8nb+n][32kp+16+k] (high nibble), two's-complement nibbles."""
    t = Wq.reshape(N // 8, K // 32, 8, 16)
    lo = (t & 0xF).astype(np.int16)
    hi = (t >> 4).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    W = np.empty((N // 8, 8, K // 32, 32), np.int16)
    W[:, :, :, :16] = lo.transpose(0, 2, 1, 3)
    W[:, :, :, 16:] = hi.transpose(0, 2, 1, 3)
    return W.reshape(N, K).astype(np.int8)


def unpack_int8(Wp, N, K):
    t = Wp.reshape(N // 8, K // 16, 8, 16)
    return t.transpose(0, 2, 1, 3).reshape(N, K)


@pytest.mark.parametrize("N,K", [(8, 32), (16, 64), (4864, 896), (24, 4096)])
def test_packers_match_oracle_and_layout(N, K):
    W, _ = q4_gemv_inputs(N, K, 1, seed=11 + N)
    q4 = x100hip.pack_w(True, W)
    assert np.array_equal(q4, ol.pack_w(True, W))
    assert np.array_equal(unpack_int4(q4, N, K), W)
    W8 = synth.rand_int8(12 + N, (N, K))
    q8 = x100hip.pack_w(False, W8)
    assert np.array_equal(q8, ol.pack_w(False, W8))
    assert np.array_equal(unpack_int8(q8, N, K), W8)


def test_oracle_gemv_known_answers():
    # closed forms: ones . ones = K; a one-hot x picks a column of W; int4 extremes
    N, K = 16, 64
    W = np.ones((N, K), np.int8)
    x = np.ones((1, K), np.int8)
    assert np.all(ol.gemv_int(W, x) == K)
    W, _ = q4_gemv_inputs(N, K, 1, seed=5)
    x = np.zeros((3, K), np.int8)
    x[0, 7] = 1
    x[1, 63] = -128
    x[2, :] = 127
    y = ol.gemv_int(W, x)
    assert np.array_equal(y[0], W[:, 7].astype(np.int32))
    assert np.array_equal(y[1], -128 * W[:, 63].astype(np.int32))
    assert np.array_equal(y[2], 127 * W.astype(np.int32).sum(1))


def test_tile_bytes_and_bad_dims():
    assert x100hip.tile_bytes(True, 4864, 896) == 4864 * 896 // 2
    assert x100hip.tile_bytes(False, 4864, 896) == 4864 * 896
    assert x100hip.tile_bytes(True, 4864, 912) == 0      # K % 32
    assert x100hip.tile_bytes(False, 12, 64) == 0        # N % 8
    with pytest.raises(x100hip.X100Error):
        x100hip.pack_w(True, np.zeros((8, 48), np.int8))


def gpu_gemv(int4, W, x, dev):
    import torch
    N, K = W.shape
    M = x.shape[0]
    s = torch.cuda.current_stream().cuda_stream
    dw = torch.from_numpy(x100hip.pack_w(int4, W).view(np.uint8)).to(dev)
    dx = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    dy = torch.full((M, N), -1, dtype=torch.int32, device=dev)
    x100hip.gemv_tile(int4, M, N, K, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
    torch.cuda.synchronize()
    return dy.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("int4", [True, False])
@pytest.mark.parametrize("N,K,M", [(4864, 896, 1), (4864, 896, 4), (4864, 896, 8), (8, 32, 1), (8, 32, 8),
                                   (40, 96, 3), (2048, 768, 2), (768, 2048, 5), (136, 4096, 1),
                                   (16, 6144, 8), (8192, 512, 3)])
def test_gemv_tile_gpu(dev, int4, N, K, M):
    if int4:
        W, x = q4_gemv_inputs(N, K, M, seed=N + K + M)
    else:
        W = synth.rand_int8(N + K, (N, K))
        x = synth.rand_int8(N + K + 1, (M, K))
    got = gpu_gemv(int4, W, x, dev)
    ref = ol.gemv_int(W, x)
    assert np.array_equal(got, ref), "int4=%s N=%d K=%d M=%d: %d mismatches" % (
        int4, N, K, M, int((got != ref).sum()))


@pytest.mark.gpu
def test_gemv_tile_extremes(dev):
    # all weights -8 (int4) / -128 (int8) and x = -128: largest magnitude sums
    N, K, M = 64, 6144, 8
    W = np.full((N, K), -8, np.int8)
    x = np.full((M, K), -128, np.int8)
    assert np.array_equal(gpu_gemv(True, W, x, dev), ol.gemv_int(W, x))
    W = np.full((N, K), -128, np.int8)
    assert np.array_equal(gpu_gemv(False, W, x, dev), ol.gemv_int(W, x))


@pytest.mark.gpu
def test_gemv_tile_rejects_bad_shapes(dev):
    import torch
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    p = buf.data_ptr()
    for args in [(0, 8, 32), (9, 8, 32), (1, 12, 32), (1, 8, 48), (8, 8, 8192)]:
        with pytest.raises(x100hip.X100Error):
            x100hip.gemv_tile(True, *args, p, p, p)
