// Measurement kernels for the hardware ceilings that bound libx100hip's kernels on the device it
// runs on (built into lib/libx100ceil.so, used by the benchmark; not part of the drop-in ABI):
//
//   x100ceil_mfma_i8  v_mfma_i32_32x32x32_i8 issued back to back from registers, no memory
//                     traffic in the loop: the int8 matrix-core ceiling, with the shader clock it
//                     ran at (s_memtime shader cycles over s_memrealtime's constant 100 MHz).
//                     Operands are either constants or random bytes (random operands toggle more
//                     of the multiplier array and draw more power, like real GEMM data).
//   x100ceil_stream   read-only streaming kernel, 16-byte loads, every load issued before the first
//                     is consumed: the floor of a kernel that must read `bytes` from memory.
//   x100ceil_empty    an empty kernel: the per-launch floor (in a graph, back to back).
//   x100ceil_handoff  a grid-wide release / counter / acquire handoff across one block per CU,
//                     with a bounded wait: the cost of passing results between blocks inside one
//                     kernel, against the kernel boundary it would replace.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// 8 independent accumulators per wave (an MFMA never waits for the previous one's result); with
// random operands, 4 A and 4 B registers sets cycle so consecutive MFMAs see different bytes.
template <bool RANDOM>
__global__ __launch_bounds__(512) void k_ceil_mfma(int iters, const v4i *__restrict__ ops, int *__restrict__ out,
                                                   unsigned long long *__restrict__ clk)
{
    v4i a[4], b[4];
    if constexpr (RANDOM) {
        const int t = threadIdx.x;   // ops holds 8 vectors per thread of a 512-thread block
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = ops[8 * t + i];
            b[i] = ops[8 * t + 4 + i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = v4i{1 + i, 2, 3, 4};
            b[i] = v4i{5, 6 + i, 7, 8};
        }
    }
    v16i acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i & 3], b[(i >> 1) & 3], acc[i], 0, 0, 0);
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[i][r];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// Block b reads 16-byte vectors b*nt*LPL + i*nt + t (i < LPL), all loads issued before any is used;
// one int per block out so nothing is eliminated.
template <int LPL>
__global__ __launch_bounds__(256) void k_ceil_stream(const v4i *__restrict__ w, size_t n16, int *__restrict__ out)
{
    const size_t base = (size_t)blockIdx.x * blockDim.x * LPL + threadIdx.x;
    v4i q[LPL];
#pragma unroll
    for (int i = 0; i < LPL; i++) {
        size_t idx = base + (size_t)i * blockDim.x;
        idx = idx < n16 ? idx : n16 - 1;
        q[i] = w[idx];
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < LPL; i++) s += q[i][0] ^ q[i][1] ^ q[i][2] ^ q[i][3];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    __shared__ int red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

__global__ void k_ceil_empty() {}

// Grid-wide handoff, the in-kernel alternative to a kernel boundary: every block (one per CU,
// all resident) first writes `dirty` ints of its own (results a producer would leave in its L2),
// then publishes one value, releases it at agent scope (the fence writes the XCD's dirty L2 lines
// back so that other XCDs can see them), and increments a device counter; then it waits for the
// counter to reach the grid size, acquires, and reads every block's value.  The wait is bounded:
// after spin_limit polls a block gives up and records status 2, so every wave always exits.
// times[b] = {s_memrealtime at arrival, at release of the wait} (100 MHz ticks); status[b]:
// 1 = every value seen, 2 = gave up, 3 = a value was missing.
// MODE 0: acquire load per poll.  MODE 1: relaxed polls and one acquire after the wait (one L2
// invalidate instead of one per poll).  MODE 2: no fences: the published value is stored and read
// with agent-scope atomic accesses (coherent across XCDs without an L2 writeback or invalidate),
// and the block waits for its stores (s_waitcnt) before the relaxed counter increment; the
// cheapest handoff possible for data written that way.
template <int MODE>
__global__ __launch_bounds__(256) void k_ceil_handoff(int dirty, int spin_limit, unsigned *__restrict__ counter,
                                                      int *__restrict__ payload, int *__restrict__ scratch,
                                                      unsigned long long *__restrict__ times, int *__restrict__ status)
{
    const int b = blockIdx.x, G = gridDim.x, t = threadIdx.x;
    for (int i = t; i < dirty; i += 256) scratch[(size_t)b * dirty + i] = b + i;
    __syncthreads();
    __shared__ int s_ok;
    unsigned long long t0 = 0, t1 = 0;
    if (t == 0) {
        t0 = __builtin_amdgcn_s_memrealtime();
        if constexpr (MODE == 2) {
            __hip_atomic_store(&payload[b], b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            payload[b] = b + 1;
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
        int it = 0;
        if constexpr (MODE == 2) {
            while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)G && it < spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                it++;
            }
        } else if constexpr (MODE == 1) {
            while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)G && it < spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                it++;
            }
            __atomic_thread_fence(__ATOMIC_ACQUIRE);
        } else {
            while (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)G && it < spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                it++;
            }
        }
        t1 = __builtin_amdgcn_s_memrealtime();
        s_ok = it < spin_limit ? 1 : 2;
    }
    __syncthreads();
    if (s_ok == 1) {
        int miss = 0;
        for (int i = t; i < G; i += 256) miss |= __hip_atomic_load(&payload[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != i + 1;
        if (__syncthreads_or(miss) && t == 0) s_ok = 3;
        __syncthreads();
    }
    if (t == 0) {
        times[2 * b] = t0;
        times[2 * b + 1] = t1;
        status[b] = s_ok;
    }
}

}  // namespace

extern "C" {

// blocks x 512 threads, iters x 8 MFMAs per wave.  ops: 512 x 8 16-byte vectors (random == 1);
// out: blocks x 512 ints; clk: blocks x {shader cycles, 100 MHz ticks}.
__attribute__((visibility("default"))) int x100ceil_mfma_i8(int blocks, int iters, int random, const void *ops,
                                                           int *out, unsigned long long *clk, void *stream)
{
    if (blocks < 1 || iters < 1 || !out || !clk || (random && !ops)) return -1;
    if (random)
        hipLaunchKernelGGL(k_ceil_mfma<true>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, iters,
                           (const v4i *)ops, out, clk);
    else
        hipLaunchKernelGGL(k_ceil_mfma<false>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, iters,
                           (const v4i *)ops, out, clk);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Reads `bytes` (a multiple of 16, pointer 16-byte aligned) with 256-thread blocks of lpl loads
// per lane; out: one int per block ((bytes / 16 + 256 lpl - 1) / (256 lpl) ints).
__attribute__((visibility("default"))) int x100ceil_stream(const void *w, size_t bytes, int *out, int lpl,
                                                          void *stream)
{
    if (!w || !out || bytes < 16 || (bytes & 15) || ((uintptr_t)w & 15)) return -1;
    const size_t n16 = bytes / 16, per = (size_t)256 * lpl;
    const dim3 grid((unsigned)((n16 + per - 1) / per));
    hipStream_t s = (hipStream_t)stream;
    switch (lpl) {
    case 1: hipLaunchKernelGGL(k_ceil_stream<1>, grid, dim3(256), 0, s, (const v4i *)w, n16, out); break;
    case 2: hipLaunchKernelGGL(k_ceil_stream<2>, grid, dim3(256), 0, s, (const v4i *)w, n16, out); break;
    case 4: hipLaunchKernelGGL(k_ceil_stream<4>, grid, dim3(256), 0, s, (const v4i *)w, n16, out); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// One block per CU (blocks <= the CU count, so all are resident); counter must be zero, payload
// holds blocks ints, scratch blocks * dirty ints, times 2 * blocks, status blocks.
__attribute__((visibility("default"))) int x100ceil_handoff(int blocks, int dirty, int spin_limit, int mode,
                                                           unsigned *counter, int *payload, int *scratch,
                                                           unsigned long long *times, int *status, void *stream)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -3;
    if (blocks < 1 || blocks > cus || dirty < 0 || spin_limit < 1 || !counter || !payload || !times || !status ||
        (dirty && !scratch))
        return -1;
    if (mode == 2)
        hipLaunchKernelGGL(k_ceil_handoff<2>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, dirty, spin_limit,
                           counter, payload, scratch, times, status);
    else if (mode == 1)
        hipLaunchKernelGGL(k_ceil_handoff<1>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, dirty, spin_limit,
                           counter, payload, scratch, times, status);
    else if (mode == 0)
        hipLaunchKernelGGL(k_ceil_handoff<0>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, dirty, spin_limit,
                           counter, payload, scratch, times, status);
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

__attribute__((visibility("default"))) int x100ceil_empty(int blocks, int threads, void *stream)
{
    if (blocks < 1 || threads < 1 || threads > 1024) return -1;
    hipLaunchKernelGGL(k_ceil_empty, dim3(blocks), dim3(threads), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
