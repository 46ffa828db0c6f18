#!/usr/bin/env python3
"""q4_gemv: int4 / int8 tile GEMV check and timing on the GPU (mirror of bench/q4_gemv.c).

Usage: python x100-gemm_amd/q4_gemv.py [N=4864] [K=896] [M=1] [nt=1] [reps=200]

Same contract as the reference CLI (bench/q4_gemv.c:105-159): W is N x K int4 in [-7, 7], x is
M x K int8, y = W . x^T in int32; the int4 weights are packed in the reference's interlaced tile
layout (pack_w_int4) and the int8 baseline in its plain tile layout (pack_w_int8).  Both GPU
results are compared with a plain integer matmul of the unpacked matrices; every row is checked
(the reference checks row 0).  Exit status 1 on a mismatch, 2 on unsupported dims.  `nt` (host
threads of the reference) has no meaning here and is accepted for argument compatibility.
"""
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import numpy as np  # noqa: E402

import synth  # noqa: E402
import x100hip  # noqa: E402


def main(argv):
    a = [int(v) for v in argv[1:]]
    N = a[0] if len(a) > 0 else 4864
    K = a[1] if len(a) > 1 else 896
    M = a[2] if len(a) > 2 else 1
    reps = a[4] if len(a) > 4 else 200
    if N % 8 or K % 32 or not 1 <= M <= 8:
        print("need N%8, K%32 (int4 pairs 2 K-blocks), 1 <= M <= 8")
        return 2
    import torch
    dev = torch.device("cuda:0")
    r = synth.rand_bytes(7, N * K + M * K)
    W = (r[:N * K].astype(np.int32) % 15 - 7).astype(np.int8).reshape(N, K)   # int4 range
    x = r[N * K:].view(np.int8).reshape(M, K).copy()
    yr = W.astype(np.int64) @ x.astype(np.int64).T                             # [N][M]
    s = torch.cuda.current_stream().cuda_stream
    dx = torch.from_numpy(x).to(dev)
    res = {}
    for int4 in (True, False):
        dw = torch.from_numpy(x100hip.pack_w(int4, W).view(np.uint8)).to(dev)
        dy = torch.empty((M, N), dtype=torch.int32, device=dev)
        x100hip.gemv_tile(int4, M, N, K, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        y = dy.cpu().numpy().astype(np.int64)
        bad = int((y != yr.T).sum())
        for _ in range(3):
            x100hip.gemv_tile(int4, M, N, K, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            x100hip.gemv_tile(int4, M, N, K, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        res[int4] = (bad, dt, dw.numel(), y[0, :4])
    bad4, dt4, b4, s4 = res[True]
    bad8, dt8, b8, s8 = res[False]
    print("int4 GEMV %dx%d M=%d: %s (%d/%d mismatch)" % (N, K, M, "FAIL" if bad4 else "y==ref OK", bad4, M * N))
    print("int8 GEMV: %s (%d/%d mismatch)" % ("FAIL" if bad8 else "y==ref OK", bad8, M * N))
    print("samples  ref: %d %d %d %d | int8: %d %d %d %d | int4: %d %d %d %d" % (
        *[int(v) for v in yr[:4, 0]], *[int(v) for v in s8], *[int(v) for v in s4]))
    print("int4: %.4f ms/GEMV  %.1f GB/s (W=%.1fMB)   int8: %.4f ms  %.1f GB/s (W=%.1fMB)   (stream launches)" % (
        dt4 * 1e3, b4 / dt4 / 1e9, b4 / 1e6, dt8 * 1e3, b8 / dt8 / 1e9, b8 / 1e6))
    print("  int4 is %.2fx faster than int8 (bandwidth halved)" % (dt8 / dt4))
    return 1 if (bad4 or bad8) else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
