// Integer tile GEMV of the decode benchmarks (bench/q4_gemv.c, bench/moe_decode.c):
//   y[M][N] = W[N][K] . x[M][K]^T,  W int4 (two per byte) or int8,  x int8,  y int32 (exact).
//
// The weights stay in the reference's own packed layouts, so a matrix packed by its pack_w_int4 /
// pack_w_int8 (bench/q4_gemv.c:37-48, 55-62) is consumed as is:
//   int8:  [N/8][K/16][128]  byte n*16 + k of tile (nb, kb) = W[8nb + n][16kb + k];
//   int4:  [N/8][K/32][128]  byte n*16 + k of tile (nb, kp) holds W[8nb + n][32kp + k] in the
//                            low nibble and W[8nb + n][32kp + 16 + k] in the high nibble
//                            (two's-complement 4-bit values).
// One wave per 8-row N-block: lane l reads 16 bytes (row n = l % 8 of tile l / 8 of each 1 KiB
// chunk), so a wave load is 64 x 16 contiguous bytes; all chunk loads of the wave are issued
// before the first is used.  x rows sit in LDS with their 16-element sums.
//
// int4 values are handled as u ^ 8 (unsigned nibble u, so u ^ 8 = q + 8 in [0, 15]):
//   sum_k q_k x_k = sum_k (u_k ^ 8) x_k - 8 * sum_k x_k,
// with v_dot4_i32_i8 on the byte-wise (u ^ 8) values.
#include "x100_common.h"
#include "x100_internal.h"

namespace {

// x [M][K] int8 -> LDS (xs, 16-byte aligned) with per-16 sums xsum [M][K/16], 1024 vectors of 16
// bytes per pass: xload issues a pass's loads (bounds-checked buffer loads), xstore writes it.
X100_DEV void xload(rsrc_t xr, int v0, v4u (&t)[4])
{
#pragma unroll
    for (int i = 0; i < 4; i++)
        t[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, (v0 + (int)threadIdx.x + 256 * i) * 16, 0, 0);
}
// Vectors past the end go to the spare slot nv (no branch, so the loads are never sunk into one).
X100_DEV void xstore(const v4u (&t)[4], int v0, int nv, int8_t *xs, int *xsum)
{
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int v = min(v0 + (int)threadIdx.x + 256 * i, nv);
        *(v4u *)(xs + v * 16) = t[i];
        int s = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) s = dot4((int)t[i][j], 0x01010101, s);
        xsum[v] = s;
    }
}

// Sum over the 8 lanes l, l^8, l^16, ..., l^56 (same row n of the N-block).
X100_DEV int sum_stride8(int v)
{
    v += dpp_i<0x128>(0, v);         // row_ror:8 = lane (i + 8) mod 16 within a row: xor 8
    v += xor16_i(v);
    v += xor32_i(v);
    return v;
}

constexpr int CH = 4;   // 1 KiB chunks per load pass

// grid = ceil(N/8 * S / 4) blocks of 4 waves.  S waves share an N-block, each taking a contiguous
// share of its chunks (S = 2 or 4 when there are too few N-blocks to give every CU several waves);
// their int32 partial sums are added through LDS, which is exact in any order.
template <int MR, bool INT4, int S>
__global__ __launch_bounds__(256) void k_gemv_tile(int M, int N, int K, const uint8_t *__restrict__ W,
                                                   const int8_t *__restrict__ x, int32_t *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int red[4][MR][8];                     // partial sums of the S waves of an N-block
    int8_t *xs = (int8_t *)smem;                      // [M][K] + one spare 16-byte slot
    int *xsum = (int *)(smem + (size_t)M * K + 16);   // [M][K/16] + one spare
    const int lane = threadIdx.x & 63, w = wave_id();
    const int Nb = N / 8;
    const int nbk = (int)blockIdx.x * (4 / S) + w / S;   // this wave's N-block
    const int ks = w % S;                                // its share of the N-block's chunks
    const int nb = min(nbk, Nb - 1);                     // clamped: the store below is skipped
    const int tiles = INT4 ? K / 32 : K / 16;            // 128-byte tiles per N-block
    const int nch = (tiles + 7) / 8;                     // 1 KiB chunks (8 tiles)
    const int cb = ks * nch / S, ce = (ks + 1) * nch / S;
    const rsrc_t wr = buf_rsrc(W + (size_t)nb * tiles * 128, (uint32_t)tiles * 128u);
    const int n = lane & 7;

    // x pass 0, then the first weight chunks, all in flight before x is stored.
    const int nv = M * K / 16;
    const rsrc_t xr = buf_rsrc(x, (uint32_t)M * K);
    v4u xt[4];
    xload(xr, 0, xt);
    // One token row: the x loads of every wave go out before any wave's weight loads (s_barrier, no
    // wait): int4 4864 x 896 3.03 -> 2.87 us; no change with int8 weights or several rows.
    if constexpr (MR == 1) __builtin_amdgcn_s_barrier();
    v4u wv[CH];
#pragma unroll
    for (int c = 0; c < CH; c++)
        wv[c] = __builtin_amdgcn_raw_buffer_load_b128(wr, ((cb + c) * 64 + lane) * 16, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    xstore(xt, 0, nv, xs, xsum);
    for (int v0 = 1024; v0 < nv; v0 += 1024) {
        xload(xr, v0, xt);
        xstore(xt, v0, nv, xs, xsum);
    }
    __syncthreads();

    int acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0;
    for (int c0 = cb; c0 < ce; c0 += CH) {
        if (c0 > cb) {
#pragma unroll
            for (int c = 0; c < CH; c++)
                wv[c] = __builtin_amdgcn_raw_buffer_load_b128(wr, ((c0 + c) * 64 + lane) * 16, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int t = (c0 + c) * 8 + (lane >> 3);   // tile of this lane
            if (t < tiles && c0 + c < ce) {
                if (INT4) {
                    int lo[4], hi[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        lo[j] = (int)((wv[c][j] & 0x0F0F0F0Fu) ^ 0x08080808u);
                        hi[j] = (int)(((wv[c][j] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u);
                    }
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        if (m < M) {
                            const v4i xl = *(const v4i *)(xs + m * K + 32 * t);
                            const v4i xh = *(const v4i *)(xs + m * K + 32 * t + 16);
                            int s = acc[m];
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                s = dot4(lo[j], xl[j], s);
                                s = dot4(hi[j], xh[j], s);
                            }
                            acc[m] = s - 8 * (xsum[m * (K / 16) + 2 * t] + xsum[m * (K / 16) + 2 * t + 1]);
                        }
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        if (m < M) {
                            const v4i xv = *(const v4i *)(xs + m * K + 16 * t);
                            int s = acc[m];
#pragma unroll
                            for (int j = 0; j < 4; j++) s = dot4((int)wv[c][j], xv[j], s);
                            acc[m] = s;
                        }
                    }
                }
            }
        }
    }
    const bool store = nbk < Nb && lane < 8;
    if constexpr (S == 1) {
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (m < M) {
                const int v = sum_stride8(acc[m]);
                if (store) y[(size_t)m * N + nb * 8 + n] = v;
            }
        }
    } else {
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const int v = sum_stride8(acc[m]);
            if (lane < 8) red[w][m][n] = v;
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) {
                if (m < M) {
                    int v = 0;
#pragma unroll
                    for (int k = 0; k < S; k++) v += red[w + k][m][n & 7];
                    if (store) y[(size_t)m * N + nb * 8 + n] = v;
                }
            }
        }
    }
}

// Waves per N-block: enough to give the chip ~1024 waves when the matrix has few N-blocks, as long
// as every wave keeps at least 3 chunks (2 with several token rows, whose dot products dominate).
inline int tile_split(int M, int N, int nch)
{
    const int nblk = N / 8;
    const int by_waves = nblk >= 1024 ? 1 : nblk >= 512 ? 2 : 4;
    const int minch = M >= 4 ? 2 : 3;
    const int by_chunks = nch / 4 >= minch ? 4 : nch / 2 >= minch ? 2 : 1;
    return min(by_waves, by_chunks);
}

template <int MR, int S>
hipError_t launch_tile_s(bool int4, int M, int N, int K, const void *W, const int8_t *x, int32_t *y, hipStream_t s)
{
    const dim3 grid((N / 8 * S + 3) / 4);
    const size_t lds = (size_t)M * K + 16 + ((size_t)M * (K / 16) + 1) * 4;
    if (int4)
        hipLaunchKernelGGL((k_gemv_tile<MR, true, S>), grid, dim3(256), lds, s, M, N, K, (const uint8_t *)W, x, y);
    else
        hipLaunchKernelGGL((k_gemv_tile<MR, false, S>), grid, dim3(256), lds, s, M, N, K, (const uint8_t *)W, x, y);
    return hipGetLastError();
}

template <int MR>
hipError_t launch_tile(bool int4, int M, int N, int K, const void *W, const int8_t *x, int32_t *y, hipStream_t s)
{
    const int tiles = int4 ? K / 32 : K / 16;
    switch (tile_split(M, N, (tiles + 7) / 8)) {
    case 1: return launch_tile_s<MR, 1>(int4, M, N, K, W, x, y, s);
    case 2: return launch_tile_s<MR, 2>(int4, M, N, K, W, x, y, s);
    default: return launch_tile_s<MR, 4>(int4, M, N, K, W, x, y, s);
    }
}

}  // namespace

hipError_t x100_gemv_tile_launch(int int4, int M, int N, int K, const void *W, const int8_t *x, int32_t *y,
                                 hipStream_t s)
{
    if (M < 1 || M > 8 || N < 8 || N % 8 || K < 16 || K % (int4 ? 32 : 16)) return hipErrorInvalidValue;
    if ((size_t)M * K + 16 + ((size_t)M * (K / 16) + 1) * 4 > 64 * 1024) return hipErrorInvalidValue;
    if (M == 1) return launch_tile<1>(int4 != 0, M, N, K, W, x, y, s);
    if (M <= 4) return launch_tile<4>(int4 != 0, M, N, K, W, x, y, s);
    return launch_tile<8>(int4 != 0, M, N, K, W, x, y, s);
}
