/*
 * x100_gemm.h -- int8 GEMM entry points of libx100hip (MI355X / gfx950 backend).
 *
 * Drop-in for the int8 part of the reference's include/x100_gemm.h.  Convention as there: all
 * matrices row-major and contiguous (lda = K, ldb = N, ldc = N); every GEMM computes
 * C = A*B + C (zero C first for C = A*B); int8 x int8 -> int32 with int32 accumulation, bit-exact
 * against the scalar oracle gemm_ref_i8 (src/gemm_ref.c:17-26 of the reference).
 *
 * Plain C ABI: plain pointers and sizes, streams passed as void* (a hipStream_t, or NULL for the
 * default stream).  Functions returning int return X100_OK (0) or a negative X100_E* code.
 */
#ifndef X100_HIP_GEMM_H
#define X100_HIP_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define X100_OK          0
#define X100_EINVAL     -1   /* bad shape / argument                                   */
#define X100_ENODEV     -2   /* no usable gfx950 device                                */
#define X100_EHIP       -3   /* HIP runtime error (x100_hip_strerror gives the detail)  */
#define X100_ENOMEM     -4   /* device allocation failed                               */

/* Replaces gemm_ime_i8 (reference include/x100_gemm.h:60-61, src/gemm_ime_i8.c:60-89).  Host
 * pointers; copies A, B, C to the GPU, computes C += A*B there, copies C back and returns when C
 * is valid.  Same signature and void return as the reference; on failure it prints the reason
 * to stderr and aborts (there is no CPU fallback).  The device buffers are allocated on the
 * first call, grow with the largest shape seen and are kept until the process ends; calls on one
 * device run one at a time (on a stream of the library's own, synchronised before returning). */
void gemm_ime_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C);

/* Same contract as gemm_ime_i8 but returns an error code instead of aborting. */
int gemm_hip_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C);

/* Device pointers, asynchronous on `stream` (C += A*B).  No host synchronisation.  For every
 * entry point C is int32 arithmetic modulo 2^32: from K = 2^17 a sum can leave the int32 range,
 * and it then wraps as the reference's int32 accumulation does. */
int gemm_hip_i8_dev(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC,
                    void *stream);

/* The overwrite form C = A*B of gemm_ime2_i8_st / gemm_ime2_i8_mt (reference
 * src/gemm_ime2_i8.c:102-147, which store each tile without reading C).  Device pointers,
 * asynchronous on `stream`.  The MFMA tile kernels and the generic kernel write C without reading
 * it; the split-K skinny kernels (M <= 16) add partial sums atomically, so for them C is first
 * cleared by a kernel (no hipMemsetAsync, so the call can be captured in a graph).  K = 0 leaves
 * C = 0.  The reference's pre-packed A/B layouts are not needed: A and B are row-major as above. */
int gemm_hip_i8_dev_set(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC,
                        void *stream);

/* Same as gemm_hip_i8_dev with an explicit kernel choice (0 auto, 1 256x256 MFMA tile,
 * 2 128x128 MFMA tile, 3 skinny M<=16 split-K, 4 generic, 5 256x256 tile with 4 waves,
 * 6 64x64 MFMA tile, 7 32x32 MFMA tile); variant | X100_GEMM_SET selects the overwrite form
 * C = A*B of gemm_hip_i8_dev_set.  For tests and measurement. */
#define X100_GEMM_SET   16
int gemm_hip_i8_dev_variant(int M, int N, int K, const int8_t *dA, const int8_t *dB, int32_t *dC,
                            void *stream, int variant);

/* Device capabilities: the GPU analogue of x100_detect / x100_caps_print (reference
 * include/x100_gemm.h:30-43, src/x100_caps.c:24-76). */
typedef struct {
    int    device;            /* HIP device ordinal                 */
    char   name[256];         /* marketing name                     */
    char   arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int    cu_count;          /* compute units                      */
    int    clock_khz;         /* peak engine clock                  */
    size_t hbm_bytes;         /* device memory                      */
    int    lds_bytes;         /* LDS per workgroup available        */
    int    l2_bytes;          /* L2 size reported by the runtime    */
    int    is_gfx950;         /* 1 when the kernels of this library can run */
} x100_hip_caps_t;

int  x100_hip_detect(x100_hip_caps_t *caps);
void x100_hip_caps_print(const x100_hip_caps_t *caps);

/* Text for the last HIP error seen on this thread (or for an X100_E* code). */
const char *x100_hip_strerror(int code);

#ifdef __cplusplus
}
#endif
#endif
