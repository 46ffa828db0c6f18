/*
 * x100_qgemv.h -- block-quantized dequant-GEMV entry points of libx100hip (gfx950).
 *
 * y[M][N] = W[N][K] . x[M][K]^T for M <= 8 token rows, W in ggml block formats, x and y fp32.
 * Each x row is quantized inside the call (Q8_0 for Q4_0 weights, Q8_K for Q4_K / Q3_K) with the
 * scalar path's rounding (quantize_q8_0_native, reference qwen_moe_hp.c:408-414; pack_A_q3k,
 * qwen_moe_q3k.c:612-624), each block's dot product is exact integer arithmetic, and the result
 * is scaled in fp32.
 *
 * Q8_0, Q5_K and Q6_K weights take the reference's int8 path (attn_k, attn_output and lm_head of
 * the mixed checkpoint, qwen_moe_q3k.c:1747-1768): x100q_pack dequantizes them and re-encodes
 * every 32 elements as Q8_0 (lin_new_i8, qwen_moe_q3k.c:872-886), and qgemv_hip quantizes x per
 * 32 with an fp32 scale (pack_A_i8, :420-427) and accumulates fma(dw * scale, isum, acc) per
 * block (run_i8_m1, :428-510; lin_mm_i8_x, :1075-1081).
 *
 * Replaces the reference's per-linear matmul `lin_mm(const Lin*, const float *x, float *y, ...)`
 * (qwen_moe.c:101-107, qwen_moe_hp.c:712-718) and the vendor kernel family
 * `gemm_kernel_i8i4* / i8i3k*` (reference/spacemit-backend/ime2_kernels.cpp:127-436): weights are
 * repacked once at load (as the vendor backend repacks in repack.cpp), then every call streams
 * them from HBM.
 *
 * All pointers are device pointers; stream is a hipStream_t passed as void* (NULL = default).
 */
#ifndef X100_HIP_QGEMV_H
#define X100_HIP_QGEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (reference bench/gguf_dump.c:12-13). */
#define X100_Q4_0  2
#define X100_Q8_0  8
#define X100_Q3_K 11
#define X100_Q4_K 12
#define X100_Q5_K 13
#define X100_Q6_K 14

/* Bytes of N rows x K columns in GGUF-native blocks (Q4_0 18 B / 32, Q8_0 34 B / 32, Q4_K
 * 144 B / 256, Q3_K 110 B / 256, Q5_K 176 B / 256, Q6_K 210 B / 256); 0 for an unsupported type
 * or K not a multiple of the block size. */
size_t x100q_gguf_bytes(int qtype, int N, int K);

/* Bytes of the device layout produced by x100q_pack: Q4_0 as GGUF (plus 256-byte alignment
 * padding), Q4_K / Q3_K K/256 sections of 148 / 114 bytes per row (the 6-bit scales unpacked to
 * bytes) each rounded up to 256 bytes, Q8_0 / Q5_K / Q6_K 34 bytes per 32 elements. */
size_t x100q_packed_bytes(int qtype, int N, int K);

/* Repack GGUF-native blocks (device pointer w_gguf, row n at n*row_bytes) into the device
 * layout used by qgemv_hip (w_packed, x100q_packed_bytes bytes).  Done once per weight, like the
 * reference's load-time repack (repack.cpp:292, 452, 928) and requantization (lin_new_i8,
 * qwen_moe_q3k.c:872-886, for Q8_0 / Q5_K / Q6_K). */
int x100q_pack(int qtype, int N, int K, const void *w_gguf, void *w_packed, void *stream);

/* y[M][N] = W . x^T.  1 <= M <= 8; K % 32 == 0 (Q4_0, Q8_0) or K % 256 == 0 (K-quants);
 * K <= 16384 for Q4_0 and the int8 path; x 16-byte aligned.  Asynchronous on stream. */
int qgemv_hip(int qtype, int M, int N, int K, const void *w_packed, const float *x, float *y,
              void *stream);

/* Self-check of the activation quantizer's arithmetic on the installed GPU; no counterpart in the
 * reference.  The quantizers compute amax / 127.0f, 1.0f / d and the fp16 truncation of d without
 * IEEE division; this runs those device functions over every float bit pattern in
 * [lo_bits, hi_bits] (<= 0x7f7fffff) and adds, into the device counters d_counts[0..2]
 * (zeroed by the caller), the inputs where they differ from the correctly rounded 1.0f / u, from
 * u / 127.0f and from the reference's truncating fp16 conversion.  The quantizers rely on zero
 * for 1/d over every positive d up to FLT_MAX / 127 and for amax / 127 over every positive
 * amax (the Q8_0 forms need only d >= RN(1e-6 / 127) and amax >= 1e-6).  Asynchronous on
 * stream. */
int x100q_check_quant_div(uint32_t lo_bits, uint32_t hi_bits, unsigned long long *d_counts, void *stream);

#ifdef __cplusplus
}
#endif
#endif
