#!/usr/bin/env python3
"""Qwen3-30B-A3B decode weight stream through the integer tile GEMV (bench/moe_decode.c).

The reference's run_fwd (bench/moe_decode.c:95-136) streams, per token and for each of the 48
layers, the attention projections q, k, v, o, the router and U experts x {gate, up, down}, then
the lm_head, each through its int4-interlaced (q4) or int8 (q8) tile GEMV with a barrier between
matmuls; it reports ms/token, tok/s and GB/s for M = 1 and for an M = 8 verify pass by expert
union U.  Decode is weight-bandwidth bound, so what is measured is the bytes streamed per token.

MI355X version (same matmul shapes, same bytes):
  * every layer and every expert slot has its own weights in HBM (the reference reuses one set,
    which on a 256 MB Infinity Cache would measure the cache, not HBM);
  * matmuls that read the same activation run as one launch over their stacked rows: q|k|v
    (N = 4096+512+512), the gate|up rows of all U experts (N = 2*768*U) and the downs of all U
    experts (N = 2048*U, K = 768; the reference feeds every matmul the same synthetic xt);
  * a token is 5 launches per layer + the lm_head, captured once in a HIP graph and replayed.
Weights are random bytes written on the device (any byte is a valid int4 pair / int8 value).

Usage: python x100-gemm_amd/moe_decode.py [nt] [--layers 48] [--reps 3] [--us 8,16,24,64]
(`nt`, the reference's host thread count, has no meaning here and is accepted for argument
compatibility.)
"""
import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import x100hip  # noqa: E402

# Qwen3-30B-A3B (bench/moe_decode.c:143)
H, NH, NKV, HD, N_EXP, N_ACT, MOE, VOCAB = 2048, 32, 4, 128, 128, 8, 768, 151936
QD, KVD = NH * HD, NKV * HD


def layer_shapes(U):
    """(N, K) of the launches of one layer streaming U experts."""
    return [(QD + 2 * KVD, H), (H, QD), (N_EXP, H), (2 * MOE * U, H), (H * U, MOE)]


def params_per_token(L, U):
    attn = (QD + 2 * KVD) * H + H * QD + N_EXP * H
    expert = 3 * MOE * H
    return attn * L + expert * U * L + VOCAB * H


class Stream:
    """Device weights for L layers x U experts (+ lm_head) and the captured per-token graph."""

    def __init__(self, torch, int4, M, U, L):
        self.torch, self.int4, self.M, self.U, self.L = torch, int4, M, U, L
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(1234 + U + 100 * M + (7 if int4 else 0))
        self.jobs = []
        for _ in range(L):
            for (N, K) in layer_shapes(U):
                self.jobs.append((N, K, self._weights(N, K, g)))
        self.jobs.append((VOCAB, H, self._weights(VOCAB, H, g)))
        self.x = torch.ones((M, max(QD, H)), dtype=torch.int8, device=dev)
        self.y = torch.empty((M, max(VOCAB, 2 * MOE * U, H * U)), dtype=torch.int32, device=dev)
        self.bytes = sum(x100hip.tile_bytes(int4, N, K) for (N, K, _) in self.jobs)
        self.graph = None

    def _weights(self, N, K, g):
        t = self.torch
        nbytes = x100hip.tile_bytes(self.int4, N, K)
        return t.randint(-128, 128, (nbytes,), dtype=t.int8, device="cuda:0", generator=g)

    def token(self):
        s = self.torch.cuda.current_stream().cuda_stream
        for (N, K, w) in self.jobs:
            x100hip.gemv_tile(self.int4, self.M, N, K, w.data_ptr(), self.x.data_ptr(), self.y.data_ptr(), s)

    def capture(self):
        t = self.torch
        self.token()
        t.cuda.synchronize()
        self.graph = t.cuda.CUDAGraph()
        side = t.cuda.Stream()
        with t.cuda.stream(side):
            with t.cuda.graph(self.graph, stream=side):
                self.token()
        t.cuda.synchronize()

    def ms_per_token(self, reps):
        t = self.torch
        if self.graph is None:
            self.capture()
        self.graph.replay()
        t.cuda.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            self.graph.replay()
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) / reps


def run(torch, L=48, reps=3, us=(8, 16, 24, 64), verbose=True):
    """Runs the sweep of bench/moe_decode.c:156-178; returns a dict of results."""
    out = {}
    say = print if verbose else (lambda *a, **k: None)
    say("Qwen3-30B-A3B  H=%d heads=%d/%d hd=%d experts=%d/%d moe_inter=%d L=%d vocab=%d" % (
        H, NH, NKV, HD, N_EXP, N_ACT, MOE, L, VOCAB))
    for int4 in (True, False):
        name = "q4-interlaced" if int4 else "q8"
        st = Stream(torch, int4, 1, N_ACT, L)
        ms1 = st.ms_per_token(reps)
        tot = params_per_token(L, N_ACT)
        say("\n[%s]  active params/tok = %.2fB of 30B  (%.0f MB %s/tok)" % (name, tot / 1e9, st.bytes / 1e6, name))
        say("  M=1 single-stream : %.3f ms/tok -> %.1f tok/s   (%.1f GB/s)" % (ms1, 1e3 / ms1, st.bytes / ms1 / 1e6))
        res = {"m1_ms_per_token": ms1, "m1_tok_s": 1e3 / ms1, "m1_GB_s": st.bytes / ms1 / 1e6,
               "bytes_per_token": st.bytes}
        del st
        say("  M=8 MTP verify (8 tokens/pass), by expert-union U:")
        for U in us:
            st = Stream(torch, int4, 8, min(U, N_EXP), L)
            msU = st.ms_per_token(reps)
            tps = 8.0 / msU * 1e3
            tag = "perfect overlap" if U == 8 else ("disjoint (worst)" if U == 64 else "partial overlap")
            say("     U=%-3d (%-16s): %.3f ms/pass -> %.1f tok/s  (%.1fx vs M=1, %.1f GB/s)" % (
                U, tag, msU, tps, tps / (1e3 / ms1), st.bytes / msU / 1e6))
            res["m8_u%d_ms_per_pass" % U] = msU
            res["m8_u%d_tok_s" % U] = tps
            del st
            torch.cuda.empty_cache()
        out[name] = res
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("nt", type=int, nargs="?", default=None, help="ignored (host threads of the reference)")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--us", default="8,16,24,64")
    args = ap.parse_args()
    import torch
    x100hip.lib()
    t0 = time.time()
    run(torch, L=args.layers, reps=args.reps, us=[int(u) for u in args.us.split(",")])
    print("\n(weight streaming through gemv_int4_hip / gemv_int8_hip; %.1f s)" % (time.time() - t0))


if __name__ == "__main__":
    main()
