"""Writes tests/golden/gemm_ref_i8.npz: int8 GEMM vectors whose expected outputs come from the
reference's own scalar gemm_ref_i8 (src/gemm_ref.c of the reference, compiled unmodified into
oracle/_ref/libx100ref.so by oracle/Makefile).  Run from the repo root after `make -C oracle`:

    python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "x100-gemm_amd"))
import synth  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "libx100ref.so")

# (M, N, K, seed): odd shapes, a K=1 outer product, and one extreme-value case (seed -1).
CASES = [(1, 1, 1, 11), (3, 5, 7, 12), (17, 33, 65, 13), (64, 48, 80, 14), (1, 64, 96, 15),
         (40, 1, 129, 16), (8, 256, 256, 17), (33, 40, 1, 18), (16, 16, 512, -1)]


def main():
    lib = ctypes.CDLL(REF)
    lib.gemm_ref_i8.argtypes = [ctypes.c_int] * 3 + [ctypes.c_void_p] * 3
    out = {}
    for idx, (M, N, K, seed) in enumerate(CASES):
        if seed < 0:
            A = np.full((M, K), -128, np.int8)
            B = np.full((K, N), -128, np.int8)
            C0 = np.zeros((M, N), np.int32)
        else:
            A, B = synth.gemm_inputs(M, N, K, seed)
            C0 = synth.rand_int8(seed + 7, (M, N)).astype(np.int32) * 1000
        C = C0.copy()
        lib.gemm_ref_i8(M, N, K, A.ctypes.data, B.ctypes.data, C.ctypes.data)
        out["A%d" % idx], out["B%d" % idx], out["C0_%d" % idx], out["C%d" % idx] = A, B, C0, C
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "gemm_ref_i8.npz"), **out)
    print("wrote %d cases" % len(CASES))


if __name__ == "__main__":
    main()
