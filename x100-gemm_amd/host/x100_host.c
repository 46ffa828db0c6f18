/* x100_host -- the integration guide's C code, compiled: a reference-side caller of the
 * block-quantized GEMV (the engine's lin_mm, qwen_moe.c:101-107) and of the MoE block
 * (qwen_moe.c:294-311) on top of libx100hip, driven through files so that the tests can feed it
 * the oracle's inputs and compare its outputs.
 *
 *   x100_host lin <qtype> <N> <K> <M> <w> <x> <y>
 *       w: N rows of GGUF-native blocks of type qtype (host bytes, as mmapped from a .gguf),
 *       x: M x K fp32; writes y: M x N fp32.  lin_hip_new + lin_hip_mm below.
 *   x100_host moe <M> <d> <ff> <n_exp> <n_act> <hn> <R> <Wg> <Wu> <Wd> <out> [ws|noalloc]
 *       hn: M x d fp32, R: n_exp x d fp32, Wg / Wu / Wd: the Q4_K expert tensors (ggml 3-D
 *       layout); writes out (M x d fp32), then sel (M x n_act int32), then sw (M x n_act fp32).
 *       moe_layer_hip, or moe_layer_hip_ws on a caller buffer, or moe_layer_hip_noalloc.
 *
 * Exit status 0 on success, 2 on bad arguments or files, 3 on a HIP or library error.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "x100_gemm.h"
#include "x100_moe.h"
#include "x100_qgemv.h"

static void die(const char *what, int code)
{
    fprintf(stderr, "x100_host: %s\n", what);
    exit(code);
}

static void hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) {
        fprintf(stderr, "x100_host: %s: %s\n", what, hipGetErrorString(e));
        exit(3);
    }
}

static void x100_ok(int rc, const char *what)
{
    if (rc != X100_OK) {
        fprintf(stderr, "x100_host: %s: %s\n", what, x100_hip_strerror(rc));
        exit(3);
    }
}

static void *read_file(const char *path, size_t bytes)
{
    FILE *f = fopen(path, "rb");
    if (!f) die("cannot open an input file", 2);
    void *p = malloc(bytes ? bytes : 1);
    if (fread(p, 1, bytes, f) != bytes || fgetc(f) != EOF) die("input file has the wrong size", 2);
    fclose(f);
    return p;
}

static void write_file(FILE *f, const void *p, size_t bytes)
{
    if (fwrite(p, 1, bytes, f) != bytes) die("cannot write the output file", 2);
}

static void *to_device(const void *host, size_t bytes)
{
    void *d = NULL;
    hip_ok(hipMalloc(&d, bytes ? bytes : 1), "hipMalloc");
    hip_ok(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "hipMemcpy");
    return d;
}

/* ---- integration guide, section 2: the engine's Lin on the GPU ---------------------------- */
typedef struct { int N, K, qtype; void *w; } LinHip;     /* w: device, x100q_packed_bytes */

static int lin_hip_new(LinHip *l, int qtype, int N, int K, const void *gguf_host, void *stream) {
    size_t raw = x100q_gguf_bytes(qtype, N, K), packed = x100q_packed_bytes(qtype, N, K);
    void *tmp;
    if (!raw) return X100_EINVAL;
    hipMalloc(&tmp, raw); hipMalloc(&l->w, packed);
    hipMemcpy(tmp, gguf_host, raw, hipMemcpyHostToDevice);
    int rc = x100q_pack(qtype, N, K, tmp, l->w, stream);   /* once, like repack.cpp */
    hipStreamSynchronize((hipStream_t)stream); hipFree(tmp);
    l->N = N; l->K = K; l->qtype = qtype;
    return rc;
}
/* y[M][N] = W . x[M][K]^T, M <= 8 rows; dx, dy device fp32 */
static int lin_hip_mm(const LinHip *l, int M, const float *dx, float *dy, void *stream) {
    return qgemv_hip(l->qtype, M, l->N, l->K, l->w, dx, dy, stream);
}

static int cmd_lin(int argc, char **argv)
{
    if (argc != 9) die("usage: x100_host lin <qtype> <N> <K> <M> <w> <x> <y>", 2);
    const int qtype = atoi(argv[2]), N = atoi(argv[3]), K = atoi(argv[4]), M = atoi(argv[5]);
    const size_t wb = x100q_gguf_bytes(qtype, N, K);
    if (!wb || M < 1 || M > 8) die("unsupported type or shape", 2);
    void *w = read_file(argv[6], wb);
    float *x = (float *)read_file(argv[7], (size_t)M * K * 4);
    hipStream_t s;
    hip_ok(hipStreamCreate(&s), "hipStreamCreate");
    LinHip l;
    x100_ok(lin_hip_new(&l, qtype, N, K, w, s), "lin_hip_new");
    float *dx = (float *)to_device(x, (size_t)M * K * 4), *dy = NULL;
    hip_ok(hipMalloc((void **)&dy, (size_t)M * N * 4), "hipMalloc");
    x100_ok(lin_hip_mm(&l, M, dx, dy, s), "lin_hip_mm");
    float *y = (float *)malloc((size_t)M * N * 4);
    hip_ok(hipMemcpyAsync(y, dy, (size_t)M * N * 4, hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    FILE *f = fopen(argv[8], "wb");
    if (!f) die("cannot create the output file", 2);
    write_file(f, y, (size_t)M * N * 4);
    fclose(f);
    hipFree(dx); hipFree(dy); hipFree(l.w); hipStreamDestroy(s);
    free(w); free(x); free(y);
    return 0;
}

/* ---- integration guide, section 4: the MoE block ------------------------------------------ */
static int cmd_moe(int argc, char **argv)
{
    if (argc != 13 && argc != 14)
        die("usage: x100_host moe <M> <d> <ff> <n_exp> <n_act> <hn> <R> <Wg> <Wu> <Wd> <out> [ws|noalloc]", 2);
    const int M = atoi(argv[2]), d = atoi(argv[3]), ff = atoi(argv[4]), n_exp = atoi(argv[5]), n_act = atoi(argv[6]);
    const char *mode = argc == 14 ? argv[13] : "";
    const size_t ws_bytes = moe_layer_workspace_bytes(M, d, ff, n_exp, n_act);
    if (!ws_bytes) die("unsupported MoE shape", 2);
    const size_t gub = x100q_gguf_bytes(X100_Q4_K, n_exp * ff, d), dnb = x100q_gguf_bytes(X100_Q4_K, n_exp * d, ff);
    float *hn = (float *)read_file(argv[7], (size_t)M * d * 4), *R = (float *)read_file(argv[8], (size_t)n_exp * d * 4);
    void *Wg = read_file(argv[9], gub), *Wu = read_file(argv[10], gub), *Wd = read_file(argv[11], dnb);
    float *d_hn = (float *)to_device(hn, (size_t)M * d * 4), *d_R = (float *)to_device(R, (size_t)n_exp * d * 4);
    void *d_Wg = to_device(Wg, gub), *d_Wu = to_device(Wu, gub), *d_Wd = to_device(Wd, dnb);
    float *d_h = NULL, *d_sw = NULL;
    int *d_sel = NULL;
    void *d_ws = NULL;
    hip_ok(hipMalloc((void **)&d_h, (size_t)M * d * 4), "hipMalloc");
    hip_ok(hipMalloc((void **)&d_sel, (size_t)M * n_act * 4), "hipMalloc");
    hip_ok(hipMalloc((void **)&d_sw, (size_t)M * n_act * 4), "hipMalloc");
    hipStream_t stream;
    hip_ok(hipStreamCreate(&stream), "hipStreamCreate");
    if (strcmp(mode, "ws") == 0) {
        hip_ok(hipMalloc(&d_ws, ws_bytes), "hipMalloc");
        hip_ok(hipMemset(d_ws, 0xFF, ws_bytes), "hipMemset");   /* any contents will do */
        x100_ok(moe_layer_hip_ws(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_h, /*residual=*/0,
                                 d_sel, d_sw, d_ws, ws_bytes, stream), "moe_layer_hip_ws");
    } else if (strcmp(mode, "noalloc") == 0) {
        x100_ok(moe_layer_hip_noalloc(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_h, /*residual=*/0,
                                      d_sel, d_sw, stream), "moe_layer_hip_noalloc");
    } else if (mode[0] == 0) {
        /* hn: [M][d] normalised hidden rows (device fp32); R: [n_exp][d] router (device fp32)
         * Wg, Wu: [n_exp][ff][d/256] Q4_K; Wd: [n_exp][d][ff/256] Q4_K (device, 16-byte aligned)
         * out: [M][d]; residual = 1 adds into out (h += eout), 0 overwrites (eout)            */
        x100_ok(moe_layer_hip(M, d, ff, n_exp, n_act, d_hn, d_R, d_Wg, d_Wu, d_Wd, d_h, /*residual=*/0,
                              d_sel, d_sw, stream), "moe_layer_hip");
    } else {
        die("mode must be ws or noalloc", 2);
    }
    float *out = (float *)malloc((size_t)M * d * 4), *sw = (float *)malloc((size_t)M * n_act * 4);
    int *sel = (int *)malloc((size_t)M * n_act * 4);
    hip_ok(hipMemcpyAsync(out, d_h, (size_t)M * d * 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip_ok(hipMemcpyAsync(sel, d_sel, (size_t)M * n_act * 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip_ok(hipMemcpyAsync(sw, d_sw, (size_t)M * n_act * 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
    FILE *f = fopen(argv[12], "wb");
    if (!f) die("cannot create the output file", 2);
    write_file(f, out, (size_t)M * d * 4);
    write_file(f, sel, (size_t)M * n_act * 4);
    write_file(f, sw, (size_t)M * n_act * 4);
    fclose(f);
    hipFree(d_hn); hipFree(d_R); hipFree(d_Wg); hipFree(d_Wu); hipFree(d_Wd); hipFree(d_h); hipFree(d_sel);
    hipFree(d_sw); hipFree(d_ws); hipStreamDestroy(stream);
    free(hn); free(R); free(Wg); free(Wu); free(Wd); free(out); free(sel); free(sw);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc >= 2 && strcmp(argv[1], "lin") == 0) return cmd_lin(argc, argv);
    if (argc >= 2 && strcmp(argv[1], "moe") == 0) return cmd_moe(argc, argv);
    die("usage: x100_host lin ... | x100_host moe ...", 2);
    return 2;
}
