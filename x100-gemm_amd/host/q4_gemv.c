/* q4_gemv -- int4 / int8 tile GEMV on the GPU, with the command line, output lines and exit
 * status of the reference's bench/q4_gemv.c:105-159.
 *
 *   usage: q4_gemv [N=4864] [K=896] [M=1] [nt=1] [reps=200]
 *
 * W is N x K int4 in [-7, 7] and x is M x K int8, drawn as the reference draws them (srand(7),
 * then rand() % 15 - 7 for W and rand() % 256 - 128 for x, bench/q4_gemv.c:114-115), packed in the
 * reference's tile layouts (x100_pack_w_int4 / x100_pack_w_int8, the byte layouts of pack_w_int4 /
 * pack_w_int8), multiplied on the GPU by gemv_int4_hip / gemv_int8_hip and compared with a plain
 * integer matmul (ref_gemv, :101-103) on every element of every row (the reference compares row 0).
 * Timing: reps back-to-back launches on one stream between two HIP events.  nt, the reference's
 * host thread count, is accepted and ignored.  Exit status 0 when both products match, 1 on a
 * mismatch, 2 on unsupported dims (N % 8, K % 32, M outside 1..8), 3 on a HIP or library error.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "x100_gemm.h"
#include "x100_gemv_tile.h"

#define HIP_OK(call)                                                                     \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) {                                                          \
            fprintf(stderr, "q4_gemv: %s failed: %s\n", #call, hipGetErrorString(e_));    \
            exit(3);                                                                     \
        }                                                                                \
    } while (0)
#define X100_OK_(call)                                                                   \
    do {                                                                                 \
        int rc_ = (call);                                                                \
        if (rc_ != X100_OK) {                                                            \
            fprintf(stderr, "q4_gemv: %s failed: %s\n", #call, x100_hip_strerror(rc_));   \
            exit(3);                                                                     \
        }                                                                                \
    } while (0)

static void ref_gemv(int M, int N, int K, const int8_t *W, const int8_t *x, int32_t *y)
{
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            int32_t a = 0;
            for (int k = 0; k < K; k++) a += (int32_t)W[(size_t)n * K + k] * (int32_t)x[(size_t)m * K + k];
            y[(size_t)m * N + n] = a;
        }
}

/* Runs one packed layout: checks every output against yr, then times reps launches. */
static int run(int int4, int M, int N, int K, const void *Wt, size_t wbytes, const int8_t *dx, const int32_t *yr,
               int reps, double *ms, int32_t sample[4])
{
    void *dw = NULL;
    int32_t *dy = NULL;
    hipStream_t s;
    hipEvent_t e0, e1;
    HIP_OK(hipStreamCreate(&s));
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipMalloc(&dw, wbytes));
    HIP_OK(hipMalloc((void **)&dy, (size_t)M * N * sizeof(int32_t)));
    HIP_OK(hipMemcpy(dw, Wt, wbytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemset(dy, 0xAB, (size_t)M * N * sizeof(int32_t)));
    if (int4) X100_OK_(gemv_int4_hip(M, N, K, (const uint8_t *)dw, dx, dy, s));
    else X100_OK_(gemv_int8_hip(M, N, K, (const int8_t *)dw, dx, dy, s));
    HIP_OK(hipStreamSynchronize(s));
    int32_t *y = (int32_t *)malloc((size_t)M * N * sizeof(int32_t));
    HIP_OK(hipMemcpy(y, dy, (size_t)M * N * sizeof(int32_t), hipMemcpyDeviceToHost));
    int bad = 0;
    for (size_t i = 0; i < (size_t)M * N; i++) bad += y[i] != yr[i];
    for (int i = 0; i < 4; i++) sample[i] = i < N ? y[i] : 0;
    free(y);
    for (int r = 0; r < 3; r++) {   /* warm-up */
        if (int4) X100_OK_(gemv_int4_hip(M, N, K, (const uint8_t *)dw, dx, dy, s));
        else X100_OK_(gemv_int8_hip(M, N, K, (const int8_t *)dw, dx, dy, s));
    }
    HIP_OK(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) {
        if (int4) X100_OK_(gemv_int4_hip(M, N, K, (const uint8_t *)dw, dx, dy, s));
        else X100_OK_(gemv_int8_hip(M, N, K, (const int8_t *)dw, dx, dy, s));
    }
    HIP_OK(hipEventRecord(e1, s));
    HIP_OK(hipEventSynchronize(e1));
    float t = 0.0f;
    HIP_OK(hipEventElapsedTime(&t, e0, e1));
    *ms = (double)t / reps;
    HIP_OK(hipFree(dw));
    HIP_OK(hipFree(dy));
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    HIP_OK(hipStreamDestroy(s));
    return bad;
}

int main(int argc, char **argv)
{
    int N = argc > 1 ? atoi(argv[1]) : 4864, K = argc > 2 ? atoi(argv[2]) : 896;
    int M = argc > 3 ? atoi(argv[3]) : 1, reps = argc > 5 ? atoi(argv[5]) : 200;
    if (N <= 0 || K <= 0 || N % 8 || K % 32 || M < 1 || M > 8) {
        printf("need N%%8,K%%32 (int4 pairs 2 K-blocks), 1 <= M <= 8\n");
        return 2;
    }
    if (reps < 1) reps = 1;
    x100_hip_caps_t caps;
    X100_OK_(x100_hip_detect(&caps));
    int8_t *W = (int8_t *)malloc((size_t)N * K), *x = (int8_t *)malloc((size_t)M * K);
    srand(7);
    for (size_t i = 0; i < (size_t)N * K; i++) W[i] = (int8_t)(rand() % 15 - 7);   /* int4 range */
    for (size_t i = 0; i < (size_t)M * K; i++) x[i] = (int8_t)(rand() % 256 - 128);
    const size_t b4 = x100_tile_bytes(1, N, K), b8 = x100_tile_bytes(0, N, K);
    uint8_t *Wq = (uint8_t *)malloc(b4);
    int8_t *Wp = (int8_t *)malloc(b8);
    X100_OK_(x100_pack_w_int4(N, K, W, Wq));
    X100_OK_(x100_pack_w_int8(N, K, W, Wp));
    int32_t *yr = (int32_t *)malloc((size_t)M * N * sizeof(int32_t));
    ref_gemv(M, N, K, W, x, yr);

    int8_t *dx = NULL;
    HIP_OK(hipMalloc((void **)&dx, (size_t)M * K));
    HIP_OK(hipMemcpy(dx, x, (size_t)M * K, hipMemcpyHostToDevice));
    double ms4 = 0, ms8 = 0;
    int32_t s4[4], s8[4];
    const int bad4 = run(1, M, N, K, Wq, b4, dx, yr, reps, &ms4, s4);
    const int bad8 = run(0, M, N, K, Wp, b8, dx, yr, reps, &ms8, s8);
    printf("int4 GEMV %dx%d M=%d: %s (%d/%d mismatch)\n", N, K, M, bad4 ? "FAIL" : "y==ref OK", bad4, M * N);
    printf("int8 GEMV: %s (%d/%d mismatch)\n", bad8 ? "FAIL" : "y==ref OK", bad8, M * N);
    printf("samples  ref: %d %d %d %d | int8: %d %d %d %d | int4: %d %d %d %d\n", yr[0], N > 1 ? yr[1] : 0,
           N > 2 ? yr[2] : 0, N > 3 ? yr[3] : 0, s8[0], s8[1], s8[2], s8[3], s4[0], s4[1], s4[2], s4[3]);
    printf("int4: %.4f ms/GEMV  %.1f GB/s (W=%.1fMB)   int8: %.4f ms  %.1f GB/s (W=%.1fMB)   %s\n", ms4,
           b4 / ms4 / 1e6, b4 / 1e6, ms8, b8 / ms8 / 1e6, b8 / 1e6, caps.name);
    printf("  int4 is %.2fx faster than int8 (bandwidth halved)\n", ms8 / ms4);
    HIP_OK(hipFree(dx));
    free(W); free(x); free(Wq); free(Wp); free(yr);
    return (bad4 || bad8) ? 1 : 0;
}
