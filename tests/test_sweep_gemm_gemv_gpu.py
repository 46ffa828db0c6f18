"""The int8 GEMM and the block-quantized GEMVs on seeded random shapes against the oracle, bit for
bit: GEMM M, N, K from 1 to 1536 (aligned and unaligned, so every kernel path, C += A.B on a
random C), GEMV Q4_0 / Q4_K / Q3_K with N up to 5000, K up to 8192 and 1 to 8 token rows."""
import numpy as np
import pytest

import oracle_lib as ol
import synth
import x100hip

pytestmark = pytest.mark.gpu


def gemm_shapes(seed=77, n=16):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        kind = int(rng.integers(0, 3))
        if kind == 0:    # multiples of the tiles
            M, N, K = (int(rng.choice([256, 512, 1024, 1536])) for _ in range(3))
        elif kind == 1:  # skinny rows
            M, N, K = int(rng.integers(1, 17)), int(rng.choice([128, 512, 1024])), int(rng.choice([512, 1024, 1536]))
        else:            # anything
            M, N, K = int(rng.integers(1, 700)), int(rng.integers(1, 700)), int(rng.integers(1, 1100))
        out.append((M, N, K, int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("M,N,K,seed", gemm_shapes())
def test_gemm_random_shape(dev, M, N, K, seed):
    import torch
    A, B = synth.gemm_inputs(M, N, K, seed=seed)
    C0 = synth.rand_int8(seed + 1, (M, N)).astype(np.int32) * 131
    dA = torch.from_numpy(np.ascontiguousarray(A)).to(dev)
    dB = torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    dC = torch.from_numpy(C0.copy()).to(dev)
    x100hip.gemm_dev(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), torch.cuda.current_stream().cuda_stream,
                     x100hip.GEMM_AUTO)
    torch.cuda.synchronize()
    ref = C0.copy()
    ol.gemm_ref_i8(A, B, ref, threads=16)
    assert np.array_equal(dC.cpu().numpy(), ref)


def gemv_shapes(seed=91, n=18):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        qt = [synth.Q4_0, synth.Q4_K, synth.Q3_K][int(rng.integers(0, 3))]
        qk = 32 if qt == synth.Q4_0 else 256
        K = qk * int(rng.integers(1, 8192 // qk + 1))
        N = int(rng.integers(1, 5001))
        out.append((qt, N, K, int(rng.integers(1, 9)), int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("qtype,N,K,M,seed", gemv_shapes())
def test_qgemv_random_shape(dev, qtype, N, K, M, seed):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    W = synth.quant_weight(qtype, N, K, seed)
    x = synth.normal_f32(seed + 1, (M, K))
    raw = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
    packed = torch.empty(x100hip.packed_bytes(qtype, N, K), dtype=torch.uint8, device=dev)
    x100hip.pack(qtype, N, K, raw.data_ptr(), packed.data_ptr(), s)
    dx = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
    dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    x100hip.qgemv(qtype, M, N, K, packed.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
    torch.cuda.synchronize()
    got = dy.cpu().numpy()
    ref = ol.qgemv(qtype, W, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "%d elements differ" % int(
        (got.view(np.uint32) != ref.view(np.uint32)).sum())
