#!/usr/bin/env python3
"""Benchmark of the quantized matrix-product path on one MI355X.

One step = one int8 GEMM C += A.B at M = N = K = 4096 (i.i.d. uniform int8 inputs, seed 2026),
inputs resident in HBM.  `value` is TOPS = 2*M*N*K / time over `--steps` back-to-back launches
timed with HIP events on the launch stream.  The same JSON line carries:
  roofline      the GEMM kernel against the dense int8 MFMA peak (5.0 POPS), plus the HBM bytes
                per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary in profiles/ (if any),
                and the same GEMM timed over three rotating A/B/C sets of 96 MiB each (288 MiB,
                more than the 256 MB Infinity Cache holds);
  cpu_baseline  the reference's scalar gemm_ref_i8 (built from its sources into oracle/_ref, or the
                oracle's restatement when that is absent) on a bounded row sample, 1 core;
  extra         the other measured shapes: skinny 8x4096x4096 GEMM, Q4_0 / Q4_K / Q3_K GEMV at
                M = 1 and 4, the int8 path (Q6_K lm_head, Q5_K attn_output, Q8_0 attn_k of
                Qwen3-30B-A3B, requantized to Q8_0 at load), the int4 / int8 tile GEMV of
                bench/q4_gemv.c, the Qwen3-30B-A3B MoE decode layer at M = 1, 4 and 8 (decode and
                speculative verify) and at 64 and 512 token rows (verify / prefill), the whole
                decoder layer (attention + MoE, 1024 and 4096 cached positions), each beside its
                scalar CPU time, and the per-token decode weight stream of bench/moe_decode.c
                (the C program x100-gemm_amd/host/moe_decode.c, run as a child process).  GEMV and
                MoE run back-to-back in a captured graph over weight copies totalling more than
                256 MB (so the 256 MB Infinity Cache cannot hold them); single-launch latency is
                reported separately.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-extra] [--no-cpu]
       python bench.py --probe     (for rocprofv3 --pmc: `--steps` GEMM 4096^3 launches, then one
                                    256 MiB device-to-device copy as the byte-count calibration)
       python bench.py --probe-all (the same with every other kernel family in between, 3 launches
                                    each at its benchmark shape)
       python bench.py --probe --gemm-variant V [--gemm-set]
                                   (the GEMM probe with kernel choice V of gemm_hip_i8_dev_variant,
                                    or the overwrite form C = A.B)
       python bench.py --ceilings  (only the measured ceilings: int8 MFMA rate and shader clock with
                                    random and constant operands, the empty-kernel launch floor in a
                                    graph, and the streaming-read floor at the rows' byte counts)

The default run also measures those ceilings: the GEMM's roofline carries its fraction of the
measured MFMA ceiling, and every GEMV / MoE / decode row carries floor_us (the streaming kernel
reading the row's bytes, same graph setting) and floor_frac = floor_us / us.
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "x100-gemm_amd"))

import synth  # noqa: E402
import x100hip  # noqa: E402

METRIC = "int8 GEMM TOPS; Q4/Q3_K GEMV GB/s (% HBM peak); MoE decode layer µs"
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def read_traffic(kernel_key):
    """HBM bytes per launch for a kernel from profiles/traffic.txt ("key bytes" lines)."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0] == kernel_key:
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


class Timer:
    """HIP events on the current (launch) stream."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, reps, warm):
        t = self.torch
        for _ in range(warm):
            fn()
        t.cuda.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps   # microseconds per call

    def graph(self, fns, replays=3, rounds=5):
        """Capture fns back to back in one graph; microseconds per fn: the median over rounds of the
        average over replays."""
        t = self.torch
        for f in fns[:2]:
            f()
        t.cuda.synchronize()
        g = t.cuda.CUDAGraph()
        side = t.cuda.Stream()
        with t.cuda.stream(side):
            with t.cuda.graph(g, stream=side):
                for f in fns:
                    f()
        t.cuda.synchronize()
        g.replay()
        t.cuda.synchronize()
        res = []
        for _ in range(rounds):
            e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(replays):
                g.replay()
            e1.record()
            t.cuda.synchronize()
            res.append(e0.elapsed_time(e1) * 1e3 / (replays * len(fns)))
        return float(np.median(res))

    def graph_ab(self, fns_a, fns_b, rounds=5, replays=3):
        """Two captured graphs timed in alternation (rounds x replays each): the medians of their
        microseconds per fn, so that neither gains from going first on a clock that is still
        settling."""
        t = self.torch
        graphs = []
        for fns in (fns_a, fns_b):
            for f in fns[:2]:
                f()
            t.cuda.synchronize()
            g = t.cuda.CUDAGraph()
            side = t.cuda.Stream()
            with t.cuda.stream(side):
                with t.cuda.graph(g, stream=side):
                    for f in fns:
                        f()
            t.cuda.synchronize()
            g.replay()
            t.cuda.synchronize()
            graphs.append((g, len(fns)))
        res = ([], [])
        for _ in range(rounds):
            for k, (g, n) in enumerate(graphs):
                e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(replays):
                    g.replay()
                e1.record()
                t.cuda.synchronize()
                res[k].append(e0.elapsed_time(e1) * 1e3 / (replays * n))
        return float(np.median(res[0])), float(np.median(res[1]))

    def single(self, fn, reps=10):
        """Isolated-launch latency: synchronise around every call."""
        t = self.torch
        best = []
        for _ in range(reps):
            t.cuda.synchronize()
            e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            t.cuda.synchronize()
            best.append(e0.elapsed_time(e1) * 1e3)
        return float(np.median(best))


# ------------------------------------------------------------------------------------------------
# Measured ceilings (x100-gemm_amd/lib/libx100ceil.so): the int8 MFMA rate and shader clock with no
# memory traffic, the per-launch floor in a graph, and the time a plain streaming kernel needs to
# read N bytes (the floor of any kernel that must read them in one launch).
# ------------------------------------------------------------------------------------------------
class Ceilings:
    def __init__(self, torch, dev, timer):
        import ctypes
        self.torch, self.dev, self.timer = torch, dev, timer
        path = os.path.join(ROOT, "x100-gemm_amd", "lib", "libx100ceil.so")
        if not os.path.exists(path):
            raise SystemExit("libx100ceil.so is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        p, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.x100ceil_mfma_i8.argtypes = [i, i, i, p, p, p, p]
        L.x100ceil_stream.argtypes = [p, sz, p, i, p]
        L.x100ceil_empty.argtypes = [i, i, p]
        L.x100ceil_handoff.argtypes = [i, i, i, i, p, p, p, p, p, p]
        self.L = L
        self._floor = {}
        self._buf = None
        self.cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def _s(self):
        return self.torch.cuda.current_stream().cuda_stream

    def mfma(self, random, iters=20000, reps=5):
        """Back-to-back v_mfma_i32_32x32x32_i8 on every SIMD (one 8-wave block per CU): TOPS and
        the shader clock (s_memtime cycles per 100 MHz s_memrealtime tick)."""
        t = self.torch
        blocks = self.cus
        ops = t.randint(-2 ** 31, 2 ** 31 - 1, (512 * 8 * 4,), dtype=t.int32, device=self.dev)
        out = t.empty(blocks * 512, dtype=t.int32, device=self.dev)
        clk = t.zeros(blocks * 2, dtype=t.int64, device=self.dev)

        def f():
            rc = self.L.x100ceil_mfma_i8(blocks, iters, 1 if random else 0, ops.data_ptr(), out.data_ptr(),
                                         clk.data_ptr(), self._s())
            if rc:
                raise RuntimeError("x100ceil_mfma_i8 rc=%d" % rc)

        us = self.timer.run(f, reps, 1)
        c = clk.cpu().numpy().reshape(-1, 2).astype(np.float64)
        ghz = float(np.mean(c[:, 0] / c[:, 1])) * 0.1
        tops = blocks * 8 * iters * 8 * 65536.0 / us / 1e6
        return {"TOPS": tops, "clock_GHz": ghz, "us": us, "frac_of_5000": tops / PEAK_INT8_TOPS,
                "TOPS_at_2.4GHz_equivalent": tops * 2.4 / ghz}

    def handoff(self, dirty_ints, mode=0, reps=20, spin_limit=200000):
        """Grid-wide in-kernel handoff (x100ceil_handoff, one 256-thread block per CU): each block
        leaves dirty_ints ints of its own in its L2, publishes a value, releases at agent scope,
        bumps a device counter and waits (bounded) for every block.  Returns the time from the last
        block's arrival to each block's release (mean and max over blocks, median over reps)."""
        t = self.torch
        G = self.cus
        counter = t.zeros(1, dtype=t.int32, device=self.dev)
        payload = t.zeros(G, dtype=t.int32, device=self.dev)
        scratch = t.zeros(max(1, G * dirty_ints), dtype=t.int32, device=self.dev)
        times = t.zeros(2 * G, dtype=t.int64, device=self.dev)
        status = t.zeros(G, dtype=t.int32, device=self.dev)
        mean_us, max_us = [], []
        for _ in range(reps):
            counter.zero_()
            payload.zero_()
            status.zero_()
            rc = self.L.x100ceil_handoff(G, dirty_ints, spin_limit, mode, counter.data_ptr(),
                                         payload.data_ptr(),
                                         scratch.data_ptr(), times.data_ptr(), status.data_ptr(), self._s())
            if rc:
                raise RuntimeError("x100ceil_handoff rc=%d" % rc)
            t.cuda.synchronize()
            st = status.cpu().numpy()
            if not (st == 1).all():
                return {"error": "status counts %s" % np.bincount(st, minlength=4).tolist()}
            tm = times.cpu().numpy().reshape(-1, 2).astype(np.float64) * 0.01   # 100 MHz ticks -> us
            last = tm[:, 0].max()
            mean_us.append(float(np.mean(tm[:, 1] - last)))
            max_us.append(float(np.max(tm[:, 1] - last)))
        return {"dirty_bytes_per_block": 4 * dirty_ints, "blocks": G,
                "protocol": ["release fence + acquire load per poll", "release fence, relaxed polls, one acquire",
                             "no fences: atomic data stores/loads, s_waitcnt, relaxed counter"][mode],
                "release_after_last_arrival_us_mean": float(np.median(mean_us)),
                "release_after_last_arrival_us_max": float(np.median(max_us))}

    def launch_floor(self, blocks, n=64):
        f = lambda: self.L.x100ceil_empty(blocks, 256, self._s())
        return self.timer.graph([f] * n)

    def stream_floor(self, nbytes):
        """Best time (graph, back to back, over rotating slices totalling more than the 256 MB
        Infinity Cache) of the streaming kernel reading nbytes, over 1, 2, 4 loads per lane."""
        nbytes = max(16, int(nbytes) // 16 * 16)
        if nbytes in self._floor:
            return self._floor[nbytes]
        t = self.torch
        pitch = (nbytes + 255) // 256 * 256
        copies = int(300e6 // nbytes) + 1
        need = copies * pitch
        if self._buf is None or self._buf.numel() < need:
            self._buf = None
            self._buf = t.randint(0, 255, (need,), dtype=t.uint8, device=self.dev)
        out = t.empty((nbytes // 16 + 255) // 256 + 1, dtype=t.int32, device=self.dev)
        base = self._buf.data_ptr()
        best = None
        for lpl in (1, 2, 4):
            fns = [lambda c=c: self.L.x100ceil_stream(base + c * pitch, nbytes, out.data_ptr(), lpl, self._s())
                   for c in range(copies)]
            us = self.timer.graph(fns)
            best = us if best is None else min(best, us)
        self._floor[nbytes] = best
        return best

    def annotate(self, row, nbytes, us):
        """Adds the streaming floor for the row's bytes and floor_frac = floor / measured time."""
        fl = self.stream_floor(nbytes)
        row["floor_us"] = fl
        row["floor_frac"] = fl / us
        return row

    def summary(self):
        res = {"mfma_i8_random": self.mfma(True), "mfma_i8_constant": self.mfma(False)}
        res["launch_floor_us"] = {str(b): self.launch_floor(b) for b in (1, 256, 1024)}
        res["grid_handoff"] = [self.handoff(n, mode) for mode in (0, 1) for n in (0, 4096, 65536)] + \
            [self.handoff(0, 2)]
        fl = {}
        for mb in (1.12, 2.18, 5.44, 7.11, 9.47, 16.0, 22.3, 28.0, 78.7, 136.9, 331.2):
            nb = int(mb * 1e6)
            us = self.stream_floor(nb)
            fl["%.2f MB" % mb] = {"us": us, "GB/s": nb / us / 1e3, "hbm_frac": nb / us / 1e3 / PEAK_HBM_GBS}
        res["stream_floor"] = fl
        return res


# ------------------------------------------------------------------------------------------------
# CPU baseline (oracle / reference build: test infrastructure, timed here as a baseline only)
# ------------------------------------------------------------------------------------------------
def cpu_gemm_baseline(K=4096, N=4096, target_s=10.0):
    import oracle_lib as ol
    ref = ol.reference()
    kind = "reference" if ref is not None else "port"
    fn = ref.gemm_ref_i8 if ref is not None else ol.oracle().gemm_ref_i8
    A, B = synth.gemm_inputs(4096, N, K, seed=2026)

    def run(rows):
        C = np.zeros((rows, N), np.int32)
        t0 = time.perf_counter()
        fn(rows, N, K, A.ctypes.data, B.ctypes.data, C.ctypes.data)
        return time.perf_counter() - t0

    probe_rows = 8
    t = run(probe_rows)
    rows = int(max(probe_rows, min(4096, probe_rows * target_s / max(t, 1e-6))))
    t = run(rows)
    tops = 2.0 * rows * N * K / t / 1e12
    return {"value": tops, "unit": "TOPS", "cores": 1, "kind": kind,
            "sample": "gemm_ref_i8 on rows 0..%d of the 4096^3 workload (%.1f s, nproc=%d)" % (
                rows, t, os.cpu_count() or 0)}


def cpu_time(fn, min_s=0.5):
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return dt / n * 1e6   # microseconds


# ------------------------------------------------------------------------------------------------
def bench_gemm(torch, timer, dev, args, ceil=None):
    """The headline: C += A.B at 4096^3, back-to-back launches on one A/B/C set (96 MiB, which the
    256 MB Infinity Cache may hold between launches).  The same launches cycling over three
    distinct sets (288 MiB, so every launch reads A, B and C from HBM and writes C back) are
    reported beside it."""
    M = N = K = 4096
    A, B = synth.gemm_inputs(M, N, K, seed=2026)
    sets = []
    for i in range(3):
        dA = torch.from_numpy(A).to(dev)
        dB = torch.from_numpy(B).to(dev)
        dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
        sets.append((dA, dB, dC))
    s = torch.cuda.current_stream().cuda_stream

    def run(nsets, fn=x100hip.gemm_dev):
        for i in range(args.warmup):
            dA, dB, dC = sets[i % nsets]
            fn(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), s)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for i in range(args.steps):
            dA, dB, dC = sets[i % nsets]
            fn(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), s)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps, time.perf_counter() - t0

    # Clock pre-roll (untimed): the shader clock takes about 40 ms of sustained load to settle
    # (series of 30 launches from a cold start measured 178, 85, 79, 77, 74, 74, then 71 us), so
    # without it the timed steps would measure the ramp rather than the kernel.
    t_end = time.perf_counter() + args.preroll_ms / 1e3
    while time.perf_counter() < t_end:
        for _ in range(20):
            x100hip.gemm_dev(M, N, K, sets[0][0].data_ptr(), sets[0][1].data_ptr(), sets[0][2].data_ptr(), s)
        torch.cuda.synchronize()
    ms, wall = run(1)
    msr, _ = run(3)
    # the overwrite form C = A.B (gemm_hip_i8_dev_set: the tile kernel stores C without reading it)
    mss, _ = run(1, x100hip.gemm_dev_set)
    mssr, _ = run(3, x100hip.gemm_dev_set)
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    topsr = ops / (msr * 1e-3) / 1e12
    log("gemm 4096^3: %.2f us/launch  %.1f TOPS (wall %.3f s for %d steps); over 3 rotating A/B/C sets "
        "(288 MiB): %.2f us  %.1f TOPS" % (ms * 1e3, tops, wall, args.steps, msr * 1e3, topsr))
    log("gemm 4096^3 overwrite form C = A.B: %.2f us  %.1f TOPS; 3 rotating sets %.2f us  %.1f TOPS" % (
        mss * 1e3, ops / mss / 1e9, mssr * 1e3, ops / mssr / 1e9))
    traffic = read_traffic("gemm_i8_4096")
    roof = {"bound": "mfma", "achieved": tops, "peak": PEAK_INT8_TOPS, "unit": "TOPS",
            "frac": tops / PEAK_INT8_TOPS, "traffic": traffic,
            "kernel": "k_gemm_big<8, 2, true> (256x256 tile, 8 waves, 2 K stages per barrier, C += A.B)",
            "algorithmic_ops_per_launch": ops,
            "rotating_sets": {"sets": 3, "bytes": 3 * (M * K + K * N + 4 * M * N), "us": msr * 1e3,
                              "TOPS": topsr, "frac": topsr / PEAK_INT8_TOPS},
            "overwrite_form": {"entry": "gemm_hip_i8_dev_set (C = A.B, C not read)", "us": mss * 1e3,
                               "TOPS": ops / mss / 1e9, "frac": ops / mss / 1e9 / PEAK_INT8_TOPS,
                               "rotating_sets_us": mssr * 1e3, "rotating_sets_TOPS": ops / mssr / 1e9,
                               "traffic": read_traffic("gemm_i8_4096_set")}}
    if ceil is not None:
        mf = ceil.mfma(True)
        roof["measured_mfma_ceiling"] = {"TOPS": mf["TOPS"], "clock_GHz": mf["clock_GHz"],
                                         "operands": "random int8, registers only (x100ceil_mfma_i8)",
                                         "frac": tops / mf["TOPS"]}
        log("gemm 4096^3 against the measured int8 MFMA ceiling (%.0f TOPS at %.2f GHz, random operands): %.3f" % (
            mf["TOPS"], mf["clock_GHz"], tops / mf["TOPS"]))
    return ms, tops, roof


def bench_extra(torch, timer, dev, args, ceil):
    import oracle_lib as ol
    extra = {}
    s = torch.cuda.current_stream().cuda_stream

    # ---- 256^3 GEMM (the reference's own gemm_bench case; launch-bound) ------------------------
    M = N = K = 256
    A, B = synth.gemm_inputs(M, N, K, seed=2026)
    dA, dB = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
    fns = [lambda: x100hip.gemm_dev(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream) for _ in range(32)]
    us = timer.graph(fns)
    lat = timer.single(fns[0])
    Cc = np.zeros((M, N), np.int32)
    cpu_us = cpu_time(lambda: ol.oracle().gemm_ref_i8(M, N, K, A.ctypes.data, B.ctypes.data, Cc.ctypes.data))
    extra["gemm_i8_256"] = {"us": us, "TOPS": 2.0 * M * N * K / us / 1e6, "single_launch_us": lat,
                            "cpu_us_1core": cpu_us, "cpu_GOPS_1core": 2.0 * M * N * K / cpu_us / 1e3}
    log("gemm 256^3: %.2f us  %.1f TOPS (single %.2f us)  cpu %.0f us = %.2f GOP/s" % (
        us, 2.0 * M * N * K / us / 1e6, lat, cpu_us, 2.0 * M * N * K / cpu_us / 1e3))

    # ---- skinny speculative-verify GEMM -------------------------------------------------------
    M, N, K = 8, 4096, 4096
    A, B = synth.gemm_inputs(M, N, K, seed=2027)
    dA, dB = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    nb = 16
    dBs = torch.stack([torch.roll(dB, i, 0) for i in range(nb)])   # 16 x 16 MB copies
    dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
    fns = [lambda i=i: x100hip.gemm_dev(M, N, K, dA.data_ptr(), dBs[i].data_ptr(), dC.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream) for i in range(nb)]
    us = timer.graph(fns)
    lat = timer.single(fns[0])
    byts = M * K + K * N + 2 * M * N * 4
    Cc = np.zeros((M, N), np.int32)
    cpu_us = cpu_time(lambda: ol.oracle().gemm_ref_i8(M, N, K, A.ctypes.data, B.ctypes.data, Cc.ctypes.data))
    extra["gemm_i8_8x4096x4096"] = ceil.annotate({"us": us, "TOPS": 2.0 * M * N * K / us / 1e6, "GB/s": byts / us / 1e3,
                                                  "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS, "single_launch_us": lat,
                                                  "cpu_us_1core": cpu_us}, byts, us)
    log("gemm 8x4096x4096: %.2f us  %.0f GB/s (single %.2f us)" % (us, byts / us / 1e3, lat))
    del dBs

    # ---- dequant GEMV ---------------------------------------------------------------------------
    for qt, name, N, K in [(synth.Q4_0, "q4_0", 4096, 4096), (synth.Q4_K, "q4_K", 6144, 2048),
                           (synth.Q3_K, "q3_K", 6144, 2048)]:
        W = synth.quant_weight(qt, N, K, seed=100 + qt)
        raw = torch.from_numpy(W.view(np.uint8).reshape(-1)).to(dev)
        pb = x100hip.packed_bytes(qt, N, K)
        copies = int(300e6 // pb) + 1
        packs = torch.empty((copies, (pb + 255) // 256 * 256), dtype=torch.uint8, device=dev)
        for i in range(copies):
            x100hip.pack(qt, N, K, raw.data_ptr(), packs[i].data_ptr(), s)
        for M in (1, 4):
            x = synth.normal_f32(7 + M, (M, K))
            dx = torch.from_numpy(x).to(dev)
            dy = torch.empty((M, N), dtype=torch.float32, device=dev)
            fns = [lambda i=i: x100hip.qgemv(qt, M, N, K, packs[i].data_ptr(), dx.data_ptr(), dy.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream) for i in range(copies)]
            us = timer.graph(fns)
            lat = timer.single(fns[0])
            byts = raw.numel() + M * K * 4 + M * N * 4
            cpu_us = cpu_time(lambda: ol.qgemv(qt, W, x))
            key = "%s_gemv_%dx%d_m%d" % (name, N, K, M)
            extra[key] = ceil.annotate({"us": us, "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                        "single_launch_us": lat, "bytes": byts, "weight_copies": copies,
                                        "cpu_us_1core": cpu_us}, byts, us)
            log("%s: %.2f us  %.0f GB/s  (%.1f%% HBM, %.2f of the %.2f us streaming floor)  single %.2f us  cpu %.0f us" % (
                key, us, byts / us / 1e3, 100 * byts / us / 1e3 / PEAK_HBM_GBS, extra[key]["floor_frac"],
                extra[key]["floor_us"], lat, cpu_us))
        del packs, raw

    # ---- int8 path: Q6_K / Q5_K / Q8_0 weights requantized to Q8_0 at load (lin_new_i8) ----------
    # Qwen3-30B-A3B's mixed checkpoint: lm_head (output.weight) Q6_K 151936 x 2048, attn_output
    # Q5_K 2048 x 4096, attn_k Q8_0 512 x 2048.  The GEMV streams the requantized weight (34 B per
    # 32 elements, the reference's BREC_I8 records), so that is the algorithmic byte count.
    for qt, name, N, K, Ms in [(synth.Q6_K, "lm_head_q6_K", 151936, 2048, (1, 4, 8)),
                               (synth.Q5_K, "attn_output_q5_K", 2048, 4096, (1, 4)),
                               (synth.Q8_0, "attn_k_q8_0", 512, 2048, (1,))]:
        W = synth.quant_weight(qt, N, K, seed=120 + qt)
        raw = torch.from_numpy(W.view(np.uint8).reshape(-1)).to(dev)
        pb = x100hip.packed_bytes(qt, N, K)
        # at least two copies (one lm_head copy is 331 MB, two exceed the Infinity Cache twice
        # over) and at least 16 launches per graph, so replays are not separated by graph gaps
        copies = max(2, int(300e6 // pb) + 1)
        nlaunch = max(16, copies)
        packs = torch.empty((copies, (pb + 255) // 256 * 256), dtype=torch.uint8, device=dev)
        for i in range(copies):
            x100hip.pack(qt, N, K, raw.data_ptr(), packs[i].data_ptr(), s)
        del raw
        Wq8 = ol.requant_q8_0(qt, W)
        wbytes = N * (K // 32) * 34
        for M in Ms:
            x = synth.normal_f32(9 + M, (M, K))
            dx = torch.from_numpy(x).to(dev)
            dy = torch.empty((M, N), dtype=torch.float32, device=dev)
            fns = [lambda i=i: x100hip.qgemv(qt, M, N, K, packs[i % copies].data_ptr(), dx.data_ptr(),
                                             dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
                   for i in range(nlaunch)]
            us = timer.graph(fns)
            lat = timer.single(fns[0])
            byts = wbytes + M * K * 4 + M * N * 4
            cpu_us = cpu_time(lambda: ol.qgemv_q8w(Wq8, x), min_s=0.3)
            key = "%s_gemv_%dx%d_m%d" % (name, N, K, M)
            extra[key] = ceil.annotate({"us": us, "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                        "single_launch_us": lat, "bytes": byts, "weight_copies": copies,
                                        "cpu_us_1core": cpu_us}, byts, us)
            log("%s: %.2f us  %.0f GB/s  (%.1f%% HBM, %.2f of the %.2f us streaming floor)  single %.2f us  cpu %.0f us" % (
                key, us, byts / us / 1e3, 100 * byts / us / 1e3 / PEAK_HBM_GBS, extra[key]["floor_frac"],
                extra[key]["floor_us"], lat, cpu_us))
        del packs, W, Wq8

    # ---- integer tile GEMV (bench/q4_gemv.c defaults: N = 4864, K = 896) ----------------------
    N, K = 4864, 896
    r = synth.rand_bytes(77, N * K)
    Wt = (r.astype(np.int32) % 15 - 7).astype(np.int8).reshape(N, K)
    for int4 in (True, False):
        packed = x100hip.pack_w(int4, Wt)
        pb = packed.nbytes
        copies = int(300e6 // pb) + 1
        dws = torch.from_numpy(packed.view(np.uint8)).to(dev).repeat(copies, 1)
        for M in (1, 8):
            xt = synth.rand_int8(78 + M, (M, K))
            dx = torch.from_numpy(xt).to(dev)
            dy = torch.empty((M, N), dtype=torch.int32, device=dev)
            fns = [lambda i=i: x100hip.gemv_tile(int4, M, N, K, dws[i].data_ptr(), dx.data_ptr(), dy.data_ptr(),
                                                 torch.cuda.current_stream().cuda_stream) for i in range(copies)]
            us = timer.graph(fns)
            lat = timer.single(fns[0])
            byts = pb + M * K + 4 * M * N
            cpu_us = cpu_time(lambda: ol.gemv_int(Wt, xt), min_s=0.3)
            key = "%s_gemv_%dx%d_m%d" % ("int4" if int4 else "int8", N, K, M)
            extra[key] = ceil.annotate({"us": us, "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                        "single_launch_us": lat, "bytes": byts, "weight_copies": copies,
                                        "cpu_us_1core": cpu_us}, byts, us)
            log("%s: %.2f us  %.0f GB/s  floor_frac %.2f  single %.2f us  cpu %.0f us" % (
                key, us, byts / us / 1e3, extra[key]["floor_frac"], lat, cpu_us))
        del dws

    # ---- Qwen3-30B-A3B decode weight stream (bench/moe_decode.c), q4 and q8 ----------------------
    # the C host program x100-gemm_amd/bin/moe_decode, run as a child process
    exe = os.path.join(ROOT, "x100-gemm_amd", "bin", "moe_decode")
    res = subprocess.run([exe, "--layers", "48", "--reps", "3", "--us", "8,24,64", "--json"], capture_output=True,
                         text=True, timeout=600)
    if res.returncode != 0:
        raise RuntimeError("moe_decode failed: " + res.stderr[-1000:])
    md = json.loads(res.stdout.strip().splitlines()[-1])
    for name in ("q4", "q8"):
        r = md[name]
        extra["moe_decode_stream_" + name] = r
        log("moe_decode %s: M=1 %.3f ms/tok (%.1f tok/s, %.0f GB/s); M=8 U=24 %.3f ms/pass (%.1f tok/s)" % (
            name, r["m1_ms_per_token"], r["m1_tok_s"], r["m1_GB_s"], r["m8_u24_ms_per_pass"], r["m8_u24_tok_s"]))

    # ---- host-pointer drop-in gemm_ime_i8 at 4096^3 (PCIe copies + allocation included) ---------
    A, B = synth.gemm_inputs(4096, 4096, 4096, seed=2026)
    Ch = np.zeros((4096, 4096), np.int32)
    x100hip.gemm_host(A, B, Ch)
    t0 = time.perf_counter()
    x100hip.gemm_host(A, B, Ch)
    host_ms = (time.perf_counter() - t0) * 1e3
    extra["gemm_ime_i8_host_4096"] = {"ms": host_ms, "TOPS_incl_pcie": 2.0 * 4096 ** 3 / host_ms / 1e9}
    log("gemm_ime_i8 host path 4096^3: %.1f ms (PCIe copies + allocation included)" % host_ms)

    # ---- MoE decode layer ----------------------------------------------------------------------
    n_exp, d, ff, n_act = 128, 2048, 768, 8
    Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed=500)
    R = synth.moe_router(n_exp, d, seed=501)
    ggml = []
    base = [torch.from_numpy(np.ascontiguousarray(w).view(np.uint8).reshape(-1)).to(dev) for w in (Wg, Wu, Wd)]
    for li in range(3):   # 3 layers x 340 MB of experts: well beyond the 256 MB Infinity Cache
        ggml.append([b.clone() for b in base] if li else base)
    # the timed layers read the experts in the tiled layout, regrouped once at load time
    # (moe_pack_experts, like x100q_pack for the GEMV weights); the ggml layout is timed beside them
    layers = []
    for Ly in ggml:
        t = [torch.empty_like(b) for b in Ly]
        for k, (rows, K) in enumerate(((ff, d), (ff, d), (d, ff))):
            x100hip.moe_pack_experts(n_exp, rows, K, Ly[k].data_ptr(), t[k].data_ptr())
        layers.append(t)
    torch.cuda.synchronize()
    dR = torch.from_numpy(R).to(dev)
    n_h = 48
    for M in (1, 4, 8):   # decode, and speculative verify of 4 and 8 rows
        hns = synth.normal_f32(900 + M, (n_h, M, d))
        dh = torch.from_numpy(hns).to(dev)
        out = torch.empty((M, d), dtype=torch.float32, device=dev)
        sel = torch.empty((n_h, M, n_act), dtype=torch.int32, device=dev)
        # caller scratch: the graph is captured on a stream of its own (moe_layer_hip_ws)
        wsb = x100hip.moe_workspace_bytes(M, d, ff, n_exp, n_act)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

        def call(i, with_sel=False, tiled=True):
            L = (layers if tiled else ggml)[i % 3]
            x100hip.moe_layer_ws(M, d, ff, n_exp, n_act, dh[i].data_ptr(), dR.data_ptr(), L[0].data_ptr(),
                                 L[1].data_ptr(), L[2].data_ptr(), out.data_ptr(), False,
                                 sel[i].data_ptr() if with_sel else None, None, ws.data_ptr(), wsb,
                                 torch.cuda.current_stream().cuda_stream, tiled=tiled)

        for i in range(n_h):
            call(i, True)
        torch.cuda.synchronize()
        U = np.array([len(set(r.ravel().tolist())) for r in sel.cpu().numpy()])
        us, us_ggml = timer.graph_ab([lambda i=i: call(i) for i in range(n_h)],
                                    [lambda i=i: call(i, tiled=False) for i in range(n_h)])
        lat = timer.single(lambda: call(0))
        byts = float(n_exp * d * 4 + U.mean() * 3 * (ff * d // 256 * 144) + M * d * 4 * 2)
        cpu_us = cpu_time(lambda: ol.moe_layer(hns[0], R, Wg, Wu, Wd, n_act), min_s=0.3)
        key = "moe_layer_qwen3_30b_a3b_m%d" % M
        extra[key] = ceil.annotate({"us_per_layer": us, "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                    "single_launch_us": lat, "experts_union_mean": float(U.mean()),
                                    "bytes_per_layer": byts, "cpu_us_1core": cpu_us, "expert_layout": "tiled",
                                    "ggml_layout_us_per_layer": us_ggml}, byts, us)
        log("%s: %.2f us/layer  U=%.1f  %.0f GB/s (%.1f%% HBM)  single %.2f us  cpu %.0f us  (ggml layout %.2f us)" % (
            key, us, U.mean(), byts / us / 1e3, 100 * byts / us / 1e3 / PEAK_HBM_GBS, lat, cpu_us, us_ggml))
    # many token rows (verify / prefill): pairs grouped by expert in chunks of 32, matrix cores
    for M in (64, 512):
        n_h = 6
        hns = synth.normal_f32(950 + M, (n_h, M, d))
        dh = torch.from_numpy(hns).to(dev)
        out = torch.empty((M, d), dtype=torch.float32, device=dev)
        sel = torch.empty((n_h, M, n_act), dtype=torch.int32, device=dev)
        wsb = x100hip.moe_workspace_bytes(M, d, ff, n_exp, n_act)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

        def callm(i, with_sel=False, tiled=True):
            L = (layers if tiled else ggml)[i % 3]
            x100hip.moe_layer_ws(M, d, ff, n_exp, n_act, dh[i].data_ptr(), dR.data_ptr(), L[0].data_ptr(),
                                 L[1].data_ptr(), L[2].data_ptr(), out.data_ptr(), False,
                                 sel[i].data_ptr() if with_sel else None, None, ws.data_ptr(), wsb,
                                 torch.cuda.current_stream().cuda_stream, tiled=tiled)

        for i in range(n_h):
            callm(i, True)
        torch.cuda.synchronize()
        U = np.array([len(set(r.ravel().tolist())) for r in sel.cpu().numpy()])
        us, us_ggml = timer.graph_ab([lambda i=i: callm(i) for i in range(n_h)],
                                    [lambda i=i: callm(i, tiled=False) for i in range(n_h)])
        byts = float(n_exp * d * 4 + U.mean() * 3 * (ff * d // 256 * 144) + M * d * 4 * 2)
        cpu_us = cpu_time(lambda: ol.moe_layer(hns[0][:8], R, Wg, Wu, Wd, n_act), min_s=0.3) * M / 8
        key = "moe_layer_qwen3_30b_a3b_m%d" % M
        extra[key] = ceil.annotate({"us_per_layer": us, "us_per_token": us / M, "tokens_per_s": M / us * 1e6,
                                    "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                    "experts_union_mean": float(U.mean()), "bytes_per_layer": byts,
                                    "cpu_us_1core": cpu_us, "cpu_note": "8-row sample scaled to M rows",
                                    "expert_layout": "tiled", "ggml_layout_us_per_layer": us_ggml}, byts, us)
        log("%s: %.2f us/layer (%.3f us/token)  U=%.1f  %.0f GB/s (%.1f%% HBM)  cpu %.0f us  (ggml layout %.2f us)" % (
            key, us, us / M, U.mean(), byts / us / 1e3, 100 * byts / us / 1e3 / PEAK_HBM_GBS, cpu_us, us_ggml))
    del layers, ggml, base

    # ---- whole decoder layer (x100_decode_layer_hip), one token --------------------------------
    # Qwen3-30B-A3B: d 2048, 32 query / 4 KV heads of 128, attention weights as in the mixed
    # checkpoint (q, v Q3_K; k Q8_0; o Q5_K), Q4_K experts; KV cache [4][ctx][128] fp32.  Four
    # device copies of the layer (1.4 GB) rotate so the Infinity Cache cannot serve them.
    types = (synth.Q3_K, synth.Q8_0, synth.Q3_K, synth.Q5_K)
    nh, nkv, hd, ctx = 32, 4, 128, 4096
    Ld = synth.decode_layer_weights(d, nh, nkv, hd, ff, n_exp, types, seed=520)
    cfg = x100hip.LayerCfg(d, nh, nkv, hd, ff, n_exp, n_act, ctx, 1e-6, 1e6, *types)
    host_cfg = ol.LayerCfg(d, nh, nkv, hd, ff, n_exp, n_act, ctx, 1e-6, 1e6, *types)
    keep = []

    def dev_layer():
        def f32(a):
            t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
            keep.append(t)
            return t.data_ptr()

        def packed(qt, W):
            N, K = W.shape[0], W.shape[1] * synth.BLOCK_ELEMS[qt]
            raw = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
            pk = torch.empty(x100hip.packed_bytes(qt, N, K), dtype=torch.uint8, device=dev)
            x100hip.pack(qt, N, K, raw.data_ptr(), pk.data_ptr(), s)
            keep.append(pk)
            return pk.data_ptr()

        def raw(W):
            t = torch.from_numpy(np.ascontiguousarray(W).view(np.uint8).reshape(-1)).to(dev)
            keep.append(t)
            return t.data_ptr()

        kc = torch.from_numpy(synth.normal_f32(530, (nkv, ctx, hd))).to(dev)
        vc = torch.from_numpy(synth.normal_f32(531, (nkv, ctx, hd))).to(dev)
        keep.extend([kc, vc])
        return x100hip.LayerWeights(f32(Ld["attn_norm"]), f32(Ld["q_norm"]), f32(Ld["k_norm"]), f32(Ld["ffn_norm"]),
                                    packed(types[0], Ld["wq"]), packed(types[1], Ld["wk"]), packed(types[2], Ld["wv"]),
                                    packed(types[3], Ld["wo"]), f32(Ld["router"]), raw(Ld["wg"]), raw(Ld["wu"]),
                                    raw(Ld["wd"]), kc.data_ptr(), vc.data_ptr())

    lw = [dev_layer() for _ in range(4)]
    attn_bytes = sum(x100hip.packed_bytes(t, n, k) for t, n, k in
                     ((types[0], nh * hd, d), (types[1], nkv * hd, d), (types[2], nkv * hd, d), (types[3], d, nh * hd)))
    h0 = synth.normal_f32(532, (d,))
    dh = torch.from_numpy(h0).to(dev)
    dwsb = x100hip.decode_workspace_bytes(cfg)
    dws = torch.empty(dwsb, dtype=torch.uint8, device=dev)
    for pos in (1023, 4095):
        fns = [lambda i=i: x100hip.decode_layer_ws(cfg, lw[i % 4], pos, dh.data_ptr(), None, None, dws.data_ptr(),
                                                   dwsb, torch.cuda.current_stream().cuda_stream)
               for i in range(16)]
        us = timer.graph(fns)
        lat = timer.single(fns[0])
        kv_bytes = 2 * nkv * (pos + 1) * hd * 4
        byts = float(attn_bytes + kv_bytes + n_exp * d * 4 + n_act * 3 * (ff * d // 256 * 144) + 6 * d * 4)
        hk = synth.normal_f32(533, (nkv, ctx, hd))
        hv = synth.normal_f32(534, (nkv, ctx, hd))
        hh = h0.copy()
        cpu_us = cpu_time(lambda: ol.decode_layer(host_cfg, Ld, hk, hv, pos, hh), min_s=0.3)
        key = "decode_layer_qwen3_30b_a3b_pos%d" % (pos + 1)
        extra[key] = ceil.annotate({"us_per_layer": us, "GB/s": byts / us / 1e3, "hbm_frac": byts / us / 1e3 / PEAK_HBM_GBS,
                                    "single_launch_us": lat, "bytes_per_layer": byts, "kv_positions": pos + 1,
                                    "cpu_us_1core": cpu_us}, byts, us)
        log("%s: %.2f us/layer  %.0f GB/s (%.1f%% HBM)  single %.2f us  cpu %.0f us  (x48 layers: %.2f ms/token)" % (
            key, us, byts / us / 1e3, 100 * byts / us / 1e3 / PEAK_HBM_GBS, lat, cpu_us, 48 * us / 1e3))
    del lw, keep
    return extra


def probe_paths(torch, dev, s, reps=3):
    """Launches of every other kernel family at its benchmark shape, for hardware counters:
    skinny GEMM, the Q4_0 / Q4_K / Q3_K GEMVs and the int8-path GEMV of the Q6_K lm_head at M = 1
    and 4, the int4 / int8 tile GEMV at M = 1, and the MoE layer at M = 1, 4, 8 and 64 (the last
    two on the matrix-core expert GEMMs), each `reps` times on distinct weight copies."""
    M, N, K = 8, 4096, 4096
    A, B = synth.gemm_inputs(M, N, K, seed=2027)
    dA = torch.from_numpy(A).to(dev)
    dBs = [torch.from_numpy(B).to(dev).roll(i, 0) for i in range(reps)]
    dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
    for i in range(reps):
        x100hip.gemm_dev(M, N, K, dA.data_ptr(), dBs[i].data_ptr(), dC.data_ptr(), s)
    torch.cuda.synchronize()
    del dBs
    for qt, N, K in [(synth.Q4_0, 4096, 4096), (synth.Q4_K, 6144, 2048), (synth.Q3_K, 6144, 2048),
                     (synth.Q6_K, 151936, 2048)]:
        W = synth.quant_weight(qt, N, K, seed=100 + qt)
        raw = torch.from_numpy(W.view(np.uint8).reshape(-1)).to(dev)
        pb = x100hip.packed_bytes(qt, N, K)
        packs = torch.empty((reps, (pb + 255) // 256 * 256), dtype=torch.uint8, device=dev)
        for i in range(reps):
            x100hip.pack(qt, N, K, raw.data_ptr(), packs[i].data_ptr(), s)
        for M in (1, 4):
            dx = torch.from_numpy(synth.normal_f32(7 + M, (M, K))).to(dev)
            dy = torch.empty((M, N), dtype=torch.float32, device=dev)
            for i in range(reps):
                x100hip.qgemv(qt, M, N, K, packs[i].data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        del packs, raw
    N, K = 4864, 896
    Wt = (synth.rand_bytes(77, N * K).astype(np.int32) % 15 - 7).astype(np.int8).reshape(N, K)
    for int4 in (True, False):
        packed = x100hip.pack_w(int4, Wt)
        dws = torch.from_numpy(packed.view(np.uint8)).to(dev).repeat(reps, 1)
        dx = torch.from_numpy(synth.rand_int8(79, (1, K))).to(dev)
        dy = torch.empty((1, N), dtype=torch.int32, device=dev)
        for i in range(reps):
            x100hip.gemv_tile(int4, 1, N, K, dws[i].data_ptr(), dx.data_ptr(), dy.data_ptr(), s)
        torch.cuda.synchronize()
        del dws
    n_exp, d, ff, n_act = 128, 2048, 768, 8
    Wg, Wu, Wd = synth.moe_weights(n_exp, d, ff, seed=500)
    dR = torch.from_numpy(synth.moe_router(n_exp, d, seed=501)).to(dev)
    base = [torch.from_numpy(np.ascontiguousarray(w).view(np.uint8).reshape(-1)).to(dev) for w in (Wg, Wu, Wd)]
    layers = []
    for _ in range(reps):   # tiled expert copies, as the benchmark times them
        t = [torch.empty_like(b) for b in base]
        for k, (rows, K) in enumerate(((ff, d), (ff, d), (d, ff))):
            x100hip.moe_pack_experts(n_exp, rows, K, base[k].data_ptr(), t[k].data_ptr(), s)
        layers.append(t)
    del base
    for M in (1, 4, 8, 64):
        dh = torch.from_numpy(synth.normal_f32(900 + M, (reps, M, d))).to(dev)
        out = torch.empty((M, d), dtype=torch.float32, device=dev)
        for i in range(reps):
            L = layers[i]
            x100hip.moe_layer(M, d, ff, n_exp, n_act, dh[i].data_ptr(), dR.data_ptr(), L[0].data_ptr(),
                              L[1].data_ptr(), L[2].data_ptr(), out.data_ptr(), False, None, None, s,
                              tiled=True)
        torch.cuda.synchronize()


def probe(torch, dev, args):
    """Launches to read hardware counters from: GEMM 4096^3 x steps (with --probe-all, then every
    other kernel family at its benchmark shape), then a 256 MiB copy that calibrates the byte
    counters."""
    M = N = K = 4096
    A, B = synth.gemm_inputs(M, N, K, seed=2026)
    dA, dB = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    fn = x100hip.gemm_dev_set if args.gemm_set else x100hip.gemm_dev
    for _ in range(args.steps):
        fn(M, N, K, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), s, args.gemm_variant)
    torch.cuda.synchronize()
    if args.probe_all:
        del dA, dB, dC
        probe_paths(torch, dev, s)
    src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log("probe: %d x gemm 4096^3, 1 x copy of %d bytes" % (args.steps, src.numel()))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--preroll-ms", type=float, default=150.0,
                    help="untimed GEMM launches before the warmup, so the shader clock has settled")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe", action="store_true")
    ap.add_argument("--probe-all", action="store_true")
    ap.add_argument("--gemm-variant", type=int, default=0,
                    help="--probe: kernel choice of gemm_hip_i8_dev_variant (0 auto, 1 256x256 8 waves, 5 4 waves)")
    ap.add_argument("--gemm-set", action="store_true", help="--probe: the overwrite form C = A.B")
    ap.add_argument("--ceilings", action="store_true",
                    help="measure only the ceilings (MFMA rate and clock, launch and streaming floors)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this backend has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import torch

    dev = torch.device("cuda:0")
    x100hip.lib()
    caps = x100hip.caps()
    if not caps.is_gfx950:
        raise SystemExit("not a gfx950 device: %s" % caps.arch.decode())
    timer = Timer(torch)
    if args.probe or args.probe_all:
        probe(torch, dev, args)
        return
    ceil = Ceilings(torch, dev, timer)
    if args.ceilings:
        print(json.dumps({"ceilings": ceil.summary(), "device": {"name": caps.name.decode(),
                                                                 "arch": caps.arch.decode(), "cus": caps.cu_count}}),
              flush=True)
        return
    ms, tops, roof = bench_gemm(torch, timer, dev, args, ceil)
    extra = {} if args.no_extra else bench_extra(torch, timer, dev, args, ceil)
    if not args.no_extra:
        extra["ceilings"] = ceil.summary()
    cpu = None if args.no_cpu else cpu_gemm_baseline()
    line = {
        "metric": METRIC, "value": tops, "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 (int32 accumulate)", "data": "synthetic (seeded uniform int8)",
        "config": {"workload": "int8 GEMM C += A.B, M=N=K=4096, row-major, int32 out",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
        "device": {"name": caps.name.decode(), "arch": caps.arch.decode(), "cus": caps.cu_count},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
