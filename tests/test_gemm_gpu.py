"""int8 GEMM on the GPU, bit-exact against the oracle gemm_ref_i8 (C += A.B)."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def gpu_gemm(A, B, C0, dev, variant=x100hip.GEMM_AUTO, reps=1):
    import torch
    M, K = A.shape
    N = B.shape[1]
    dA = torch.from_numpy(np.ascontiguousarray(A)).to(dev)
    dB = torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    dC = torch.from_numpy(np.ascontiguousarray(C0).copy()).to(dev)
    for _ in range(reps):
        x100hip.gemm_dev(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), _stream(), variant)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


def oracle_gemm(A, B, C0, threads=16):
    C = np.ascontiguousarray(C0).copy()
    ol.gemm_ref_i8(A, B, C, threads=threads)
    return C


def test_gemm_256_cube(dev):
    A, B = synth.gemm_inputs(256, 256, 256, seed=2026)
    C0 = np.zeros((256, 256), np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))
    C0 = synth.rand_int8(1, (256, 256)).astype(np.int32) * 77
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (8, 4096, 4096), (300, 200, 96), (2048, 2048, 1024)])
def test_gemm_overwrite_form(dev, M, N, K):
    # C = A*B whatever C held before (the overwrite form of gemm_ime2_i8_st / _mt): the MFMA tiles,
    # the skinny split-K kernel (atomics into the cleared C) and the generic kernel.
    import torch
    A, B = synth.gemm_inputs(M, N, K, seed=3030 + M)
    garbage = synth.rand_int8(5, (M, N)).astype(np.int32) * 12345
    dA = torch.from_numpy(A).to(dev)
    dB = torch.from_numpy(B).to(dev)
    dC = torch.from_numpy(garbage.copy()).to(dev)
    x100hip.gemm_dev_set(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert np.array_equal(dC.cpu().numpy(), oracle_gemm(A, B, np.zeros((M, N), np.int32)))


# (variant, M, N, K): every kernel's overwrite form.  The 256x256 kernel with superstages (K / 64 a
# multiple of 8) and without (K = 576), 8 and 4 waves; the register-staged tiles with and without
# edges; the generic kernel; the skinny split-K kernels (cleared C + atomics).
SET_CASES = [(x100hip.GEMM_TILE256, 4096, 4096, 4096), (x100hip.GEMM_TILE256, 512, 768, 576),
             (x100hip.GEMM_TILE256_W4, 1024, 512, 1024), (x100hip.GEMM_TILE256_W4, 256, 512, 576),
             (x100hip.GEMM_TILE128, 384, 256, 320), (x100hip.GEMM_TILE128, 130, 144, 96),
             (x100hip.GEMM_TILE64, 256, 192, 128), (x100hip.GEMM_TILE64, 65, 80, 48),
             (x100hip.GEMM_TILE32, 96, 64, 64), (x100hip.GEMM_TILE32, 33, 48, 80),
             (x100hip.GEMM_GENERIC, 70, 50, 33), (x100hip.GEMM_SKINNY, 8, 4096, 4096),
             (x100hip.GEMM_SKINNY, 5, 272, 96)]


@pytest.mark.parametrize("variant,M,N,K", SET_CASES)
def test_gemm_overwrite_form_variants(dev, variant, M, N, K):
    # C = A*B with C holding garbage before; a second call on the result must not accumulate.
    import torch
    A, B = synth.gemm_inputs(M, N, K, seed=4040 + M + N + K)
    garbage = synth.rand_int8(6, (M, N)).astype(np.int32) * 54321
    dA = torch.from_numpy(A).to(dev)
    dB = torch.from_numpy(B).to(dev)
    dC = torch.from_numpy(garbage.copy()).to(dev)
    ref = oracle_gemm(A, B, np.zeros((M, N), np.int32))
    x100hip.gemm_dev_set(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), _stream(), variant)
    torch.cuda.synchronize()
    assert np.array_equal(dC.cpu().numpy(), ref)
    x100hip.gemm_dev_set(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), _stream(), variant)
    torch.cuda.synchronize()
    assert np.array_equal(dC.cpu().numpy(), ref)


def test_gemm_overwrite_form_k0_and_unaligned_c(dev):
    # K = 0 gives C = 0 (A and B may be null); a C 4 bytes past a 16-byte boundary takes the
    # clear's scalar head; the words around C keep their values.
    import torch
    M, N = 33, 47
    buf = torch.full((M * N + 8,), 99, dtype=torch.int32, device=dev)
    assert buf.data_ptr() % 16 == 0
    ptr = buf.data_ptr() + 4
    x100hip.gemm_dev_set(M, N, 0, 0, 0, ptr, _stream())
    torch.cuda.synchronize()
    h = buf.cpu().numpy()
    assert h[0] == 99 and np.all(h[1:1 + M * N] == 0) and np.all(h[1 + M * N:] == 99)
    A, B = synth.gemm_inputs(M, N, 64, seed=31)
    dA = torch.from_numpy(A).to(dev)
    dB = torch.from_numpy(B).to(dev)
    buf.fill_(7)
    x100hip.gemm_dev_set(M, N, 64, dA.data_ptr(), dB.data_ptr(), ptr, _stream())
    torch.cuda.synchronize()
    h = buf.cpu().numpy()
    assert h[0] == 7 and np.all(h[1 + M * N:] == 7)
    assert np.array_equal(h[1:1 + M * N].reshape(M, N), oracle_gemm(A, B, np.zeros((M, N), np.int32)))


def test_gemm_4096_cube(dev):
    A, B = synth.gemm_inputs(4096, 4096, 4096, seed=2026)
    C0 = np.zeros((4096, 4096), np.int32)
    got = gpu_gemm(A, B, C0, dev)
    ref = oracle_gemm(A, B, C0)
    assert np.array_equal(got, ref), "mismatches: %d" % int((got != ref).sum())


@pytest.mark.parametrize("variant", [x100hip.GEMM_TILE256, x100hip.GEMM_TILE256_W4])
def test_gemm_4096_cube_variants(dev, variant):
    A, B = synth.gemm_inputs(4096, 4096, 4096, seed=2028)
    C0 = synth.rand_int8(8, (4096, 4096)).astype(np.int32) * 1000
    assert np.array_equal(gpu_gemm(A, B, C0, dev, variant), oracle_gemm(A, B, C0))


def test_gemm_4096_accumulate_twice(dev):
    A, B = synth.gemm_inputs(4096, 4096, 4096, seed=7)
    C0 = np.zeros((4096, 4096), np.int32)
    once = gpu_gemm(A, B, C0, dev)
    twice = gpu_gemm(A, B, C0, dev, reps=2)
    assert np.array_equal(twice, 2 * once)


def test_gemm_skinny_8x4096x4096(dev):
    A, B = synth.gemm_inputs(8, 4096, 4096, seed=2027)
    C0 = synth.rand_int8(2, (8, 4096)).astype(np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))


@pytest.mark.parametrize("M,N,K", [(1, 128, 512), (16, 384, 1024), (7, 1152, 2560), (5, 768, 1536),
                                   (16, 2048, 8192), (2, 4096, 512)])
def test_gemm_skinny_matrix_cores(dev, M, N, K):
    # M <= 16, N % 128 == 0, K % 512 == 0: the split-K matrix-core kernel (512 x 128 B slabs)
    A, B = synth.gemm_inputs(M, N, K, seed=5 * M + N + K)
    C0 = synth.rand_int8(8, (M, N)).astype(np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))


def test_gemm_skinny_matrix_cores_extremes(dev):
    # every product -128 * -128: per element 16384 * K, the largest int8 sum
    M, N, K = 16, 256, 2048
    A = np.full((M, K), -128, np.int8)
    B = np.full((K, N), -128, np.int8)
    got = gpu_gemm(A, B, np.zeros((M, N), np.int32), dev)
    assert np.array_equal(got, np.full((M, N), 16384 * K, np.int32))


SHAPES = [(1, 16, 16), (2, 32, 48), (8, 4096, 256), (16, 272, 528), (17, 48, 80), (33, 48, 80),
          (128, 128, 64), (130, 144, 96), (255, 256, 256), (256, 256, 64), (300, 272, 1040),
          (512, 512, 512), (257, 528, 336), (1024, 768, 256)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_shapes_auto(dev, M, N, K):
    A, B = synth.gemm_inputs(M, N, K, seed=M + 3 * N + 7 * K)
    C0 = synth.rand_int8(5, (M, N)).astype(np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))


@pytest.mark.parametrize("variant", [x100hip.GEMM_TILE256, x100hip.GEMM_TILE128, x100hip.GEMM_SKINNY,
                                     x100hip.GEMM_GENERIC, x100hip.GEMM_TILE256_W4, x100hip.GEMM_TILE64,
                                     x100hip.GEMM_TILE32])
@pytest.mark.parametrize("M,N,K", [(8, 256, 256), (16, 512, 320), (3, 48, 64), (256, 256, 512),
                                   (40, 96, 144), (512, 768, 1024), (768, 512, 576)])
def test_gemm_forced_variants(dev, variant, M, N, K):
    if variant == x100hip.GEMM_SKINNY and M > 16:
        pytest.skip("skinny kernel takes M <= 16")
    A, B = synth.gemm_inputs(M, N, K, seed=11 * M + N + K)
    C0 = synth.rand_int8(6, (M, N)).astype(np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev, variant), oracle_gemm(A, B, C0))


@pytest.mark.parametrize("M,N,K", [(5, 20, 40), (64, 30, 64), (9, 17, 33), (100, 100, 100)])
def test_gemm_unaligned_shapes(dev, M, N, K):
    # K or N not a multiple of 16: row starts are not 16-byte aligned -> generic kernel
    A, B = synth.gemm_inputs(M, N, K, seed=M + N + K)
    C0 = np.zeros((M, N), np.int32)
    assert np.array_equal(gpu_gemm(A, B, C0, dev), oracle_gemm(A, B, C0))


def test_gemm_extremes(dev):
    K = 512
    A = np.full((64, K), -128, np.int8)
    B = np.full((K, 64), -128, np.int8)
    C = gpu_gemm(A, B, np.zeros((64, 64), np.int32), dev)
    assert np.all(C == 16384 * K)
    A = np.full((64, K), 127, np.int8)
    C = gpu_gemm(A, B, np.zeros((64, 64), np.int32), dev)
    assert np.all(C == -127 * 128 * K)


def test_gemm_empty_is_noop(dev):
    import torch
    dC = torch.ones((4, 4), dtype=torch.int32, device=dev)
    x100hip.gemm_dev(4, 4, 0, 0, 0, dC.data_ptr(), _stream())
    x100hip.gemm_dev(0, 4, 4, 0, 0, dC.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert int(dC.sum()) == 16


def test_gemm_host_dropin(dev):
    A, B = synth.gemm_inputs(96, 80, 64, seed=8)
    C = synth.rand_int8(9, (96, 80)).astype(np.int32)
    ref = oracle_gemm(A, B, C)
    x100hip.gemm_host(A, B, C)
    assert np.array_equal(C, ref)
    # the void drop-in entry point (reference name)
    C2 = np.zeros((96, 80), np.int32)
    x100hip.lib().gemm_ime_i8(96, 80, 64, A.ctypes.data, B.ctypes.data, C2.ctypes.data)
    assert np.array_equal(C2, oracle_gemm(A, B, np.zeros((96, 80), np.int32)))


def test_gemm_host_dropin_reuses_buffers(dev):
    # The host path keeps its device buffers between calls and grows them: a small call, a larger
    # one (the buffers grow), a smaller one again (the larger buffers hold stale data beyond it),
    # and two host threads at once (calls on one device run one at a time).
    import threading
    # (2048, 1280, 1024): C is 10 MiB, two 8 MiB staging chunks, the second partial; A and B share
    # the chunk stream with C
    for i, (M, N, K) in enumerate([(40, 48, 32), (512, 384, 256), (24, 16, 48), (256, 272, 1040),
                                   (2048, 1280, 1024), (64, 48, 16)]):
        A, B = synth.gemm_inputs(M, N, K, seed=60 + i)
        C = synth.rand_int8(61 + i, (M, N)).astype(np.int32)
        ref = oracle_gemm(A, B, C)
        x100hip.gemm_host(A, B, C)
        assert np.array_equal(C, ref), (M, N, K)
    jobs = []
    for i in range(4):
        A, B = synth.gemm_inputs(128 + 64 * i, 96, 64 * (i + 1), seed=70 + i)
        C = np.zeros((A.shape[0], 96), np.int32)
        jobs.append((A, B, C, oracle_gemm(A, B, C)))
    errs = []

    def run(job):
        try:
            x100hip.gemm_host(job[0], job[1], job[2])
        except Exception as e:   # collected and re-raised in the main thread
            errs.append(e)

    ts = [threading.Thread(target=run, args=(j,)) for j in jobs]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs
    for A, B, C, ref in jobs:
        assert np.array_equal(C, ref)


@pytest.mark.parametrize("variant,M,N", [(x100hip.GEMM_AUTO, 4, 256), (x100hip.GEMM_AUTO, 32, 256),
                                         (x100hip.GEMM_TILE256, 256, 256), (x100hip.GEMM_TILE64, 64, 128)])
def test_gemm_long_k_wraps_like_int32(dev, variant, M, N):
    # K = 2^17 + 512: all -128 inputs give K * 16384 = 2,155,872,256 per element, past 2^31; the
    # result (and C += on top of it) is the int32 wrap of the exact sum, as the reference's int32
    # accumulation gives.  A random slice is checked against an exact int64 product.
    K = (1 << 17) + 512
    A = np.full((M, K), -128, np.int8)
    B = np.full((K, N), -128, np.int8)
    C0 = np.full((M, N), 7, np.int32)
    want = np.int64(7) + np.int64(K) * 16384
    got = gpu_gemm(A, B, C0, dev, variant)
    assert np.all(got == np.int32(((want + 2**31) % 2**32) - 2**31))
    rng = np.random.default_rng(41)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    exact = A[:, :].astype(np.int64) @ B[:, :8].astype(np.int64)
    got = gpu_gemm(A, B, np.zeros((M, N), np.int32), dev, variant)
    assert np.array_equal(got[:, :8], (((exact + 2**31) % 2**32) - 2**31).astype(np.int32))


def test_gemm_rejects_bad_args(dev):
    with pytest.raises(x100hip.X100Error):
        x100hip.gemm_dev(-1, 4, 4, 1, 1, 1, _stream())
