/*
 * x100_gemv_tile.h -- integer tile GEMV of the decode benchmarks (libx100hip, gfx950).
 *
 * y[M][N] = W[N][K] . x[M][K]^T with int8 activations, int4 or int8 weights and exact int32
 * results: the contract of the reference's ref_gemv / gemv_nb_int4 / gemv_nb_int8
 * (bench/q4_gemv.c:67-103, also bench/moe_decode.c:56-88).  Weights use the reference's packed
 * layouts unchanged, so the output of its pack_w_int4 / pack_w_int8 can be uploaded as is:
 *   int4: [N/8][K/32][128] bytes, byte n*16+k of tile (nb,kp) = W[8nb+n][32kp+k] (low nibble)
 *         | W[8nb+n][32kp+16+k] << 4 (high nibble), values two's-complement 4-bit
 *         (pack_w_int4, bench/q4_gemv.c:37-48);
 *   int8: [N/8][K/16][128] bytes, byte n*16+k of tile (nb,kb) = W[8nb+n][16kb+k]
 *         (pack_w_int8, bench/q4_gemv.c:55-62).
 * x is plain row-major M x K int8 (the reference's pack_x tile copy, bench/q4_gemv.c:50-53, is
 * not needed); y is row-major M x N int32 and is overwritten.
 */
#ifndef X100_HIP_GEMV_TILE_H
#define X100_HIP_GEMV_TILE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the packed weight layout (N*K/2 for int4, N*K for int8); 0 for unsupported dims
 * (N % 8, K % 32 for int4, K % 16 for int8). */
size_t x100_tile_bytes(int int4, int N, int K);

/* Host-side packers with the reference's byte layouts (replace pack_w_int4 / pack_w_int8,
 * bench/q4_gemv.c:37-48, 55-62).  W is N x K int8 row-major (int4: values in [-8, 7]).
 * Return 0, or X100_EINVAL for unsupported dims / NULL pointers. */
int x100_pack_w_int4(int N, int K, const int8_t *W, uint8_t *Wq);
int x100_pack_w_int8(int N, int K, const int8_t *W, int8_t *Wp);

/* y = W . x^T on the device (all pointers device memory), asynchronous on stream (hipStream_t
 * as void*, NULL = default).  1 <= M <= 8; N % 8 == 0; K % 32 (int4) or K % 16 (int8);
 * M*K*1.25 <= 64 KiB.  Replaces gemv_nb_int4 / gemv_nb_int8 (bench/q4_gemv.c:67-99) over all
 * N-blocks. */
int gemv_int4_hip(int M, int N, int K, const uint8_t *Wq, const int8_t *x, int32_t *y, void *stream);
int gemv_int8_hip(int M, int N, int K, const int8_t *Wp, const int8_t *x, int32_t *y, void *stream);

#ifdef __cplusplus
}
#endif
#endif
