/* moe_decode -- the Qwen3-30B-A3B decode weight stream of the reference's bench/moe_decode.c
 * (run_fwd, :95-136; sweep, :138-185) through gemv_int4_hip / gemv_int8_hip on one GPU.
 *
 *   usage: moe_decode [nt] [--layers L] [--reps R] [--us 8,16,24,64] [--check] [--json]
 *
 * Per token and layer the reference streams q, k, v, o, the router and U experts x {gate, up,
 * down} through its int4 (q4) or int8 (q8) tile GEMV, then the lm_head; it reports ms/token, tok/s
 * and GB/s at M = 1 (U = 8) and for an M = 8 verify pass by expert union U.  Here:
 *   * every layer and expert slot has its own weights in HBM (the reference reuses one set, which
 *     on MI355X would be served by the 256 MB Infinity Cache instead of HBM);
 *   * matmuls that read the same activation are one launch over their stacked rows: q|k|v, the
 *     gate|up rows of the U experts, the downs of the U experts (5 launches per layer);
 *   * a token's launches are captured once into a HIP graph and replayed, timed between events.
 * Weight bytes are copied from a 64 MiB pool of splitmix64 bytes (any byte is a valid int4 pair
 * or int8 value); x holds random int8 rows.
 *
 * --check runs every launch of every configuration once, eagerly, and compares each output with
 * an integer matmul of the same weights on the host; after the timed graph replays it compares
 * the final launch's output (the lm_head) again.  Exit status 1 on any mismatch.  --json prints
 * the results as one JSON line at the end.  nt, the reference's thread count, is ignored.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "x100_gemm.h"
#include "x100_gemv_tile.h"

/* Qwen3-30B-A3B (bench/moe_decode.c:141-143) */
enum { H = 2048, NH = 32, NKV = 4, HD = 128, N_EXP = 128, N_ACT = 8, MOE = 768, VOCAB = 151936 };
enum { QD = NH * HD, KVD = NKV * HD, XK = QD > H ? QD : H };
#define POOL ((size_t)64 << 20)

static void hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) {
        fprintf(stderr, "moe_decode: %s: %s\n", what, hipGetErrorString(e));
        exit(3);
    }
}

static void x100_ok(int rc, const char *what)
{
    if (rc != X100_OK) {
        fprintf(stderr, "moe_decode: %s: %s\n", what, x100_hip_strerror(rc));
        exit(3);
    }
}

static uint64_t splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

typedef struct {
    int N, K;
    size_t off;       /* weight byte j is pool[(off + j) % POOL] */
    void *w;          /* device, x100_tile_bytes(int4, N, K) */
} Job;

typedef struct {
    int int4, M, U, L, njobs;
    Job *jobs;
    size_t bytes;     /* weight bytes streamed per token */
    int8_t *dx;
    int32_t *dy;
    hipStream_t s;
    hipGraphExec_t exec;
} Stream;

static const uint8_t *g_pool_host;
static const uint8_t *g_pool_dev;

static void fill(void *dst, size_t n, size_t off, hipStream_t s)
{
    size_t done = 0;
    while (done < n) {
        const size_t p = (off + done) % POOL, len = (n - done) < (POOL - p) ? (n - done) : (POOL - p);
        hip_ok(hipMemcpyAsync((uint8_t *)dst + done, g_pool_dev + p, len, hipMemcpyDeviceToDevice, s), "fill");
        done += len;
    }
}

/* Weight value W[n][k] of a job from the pool, through the tile layouts of bench/q4_gemv.c:37-62:
 * int4 tile (n/8, k/32) of 128 bytes, byte 16*(n%8) + k%16 holding k%32 < 16 in the low nibble and
 * k%32 >= 16 in the high nibble (sign-extended); int8 tile (n/8, k/16), byte 16*(n%8) + k%16. */
static int wval(const Job *j, int int4, int n, int k)
{
    if (int4) {
        const size_t t = ((size_t)(n / 8) * (j->K / 32) + k / 32) * 128 + 16 * (n % 8) + (k % 16);
        const uint8_t b = g_pool_host[(j->off + t) % POOL];
        return (k % 32) < 16 ? (int8_t)(b << 4) >> 4 : (int8_t)b >> 4;
    }
    const size_t t = ((size_t)(n / 8) * (j->K / 16) + k / 16) * 128 + 16 * (n % 8) + (k % 16);
    return (int8_t)g_pool_host[(j->off + t) % POOL];
}

static int check_job(const Stream *st, const Job *j, const int8_t *x, const char *what)
{
    int32_t *y = (int32_t *)malloc((size_t)st->M * j->N * 4);
    hip_ok(hipMemcpyAsync(y, st->dy, (size_t)st->M * j->N * 4, hipMemcpyDeviceToHost, st->s), "copy y");
    hip_ok(hipStreamSynchronize(st->s), "sync");
    long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 64)
    for (int n = 0; n < j->N; n++) {
        int w[XK];
        for (int k = 0; k < j->K; k++) w[k] = wval(j, st->int4, n, k);
        for (int m = 0; m < st->M; m++) {
            int32_t a = 0;
            for (int k = 0; k < j->K; k++) a += w[k] * (int32_t)x[(size_t)m * j->K + k];   /* rows of K */
            bad += a != y[(size_t)m * j->N + n];
        }
    }
    free(y);
    if (bad) fprintf(stderr, "moe_decode: %s: %ld of %ld outputs differ (N=%d K=%d)\n", what, bad,
                     (long)st->M * j->N, j->N, j->K);
    return bad != 0;
}

static void launch(const Stream *st, const Job *j)
{
    if (st->int4) x100_ok(gemv_int4_hip(st->M, j->N, j->K, (const uint8_t *)j->w, st->dx, st->dy, st->s), "gemv_int4_hip");
    else x100_ok(gemv_int8_hip(st->M, j->N, j->K, (const int8_t *)j->w, st->dx, st->dy, st->s), "gemv_int8_hip");
}

static void stream_init(Stream *st, int int4, int M, int U, int L, const int8_t *x, size_t *pool_off)
{
    static const int shapes[5][2] = {{0, H}, {H, QD}, {N_EXP, H}, {0, H}, {0, MOE}};
    memset(st, 0, sizeof *st);
    st->int4 = int4, st->M = M, st->U = U, st->L = L, st->njobs = 5 * L + 1;
    st->jobs = (Job *)calloc((size_t)st->njobs, sizeof(Job));
    hip_ok(hipStreamCreate(&st->s), "hipStreamCreate");
    int maxn = VOCAB;
    for (int i = 0; i < st->njobs; i++) {
        Job *j = &st->jobs[i];
        const int a = i % 5;
        if (i == 5 * L) {
            j->N = VOCAB, j->K = H;                                  /* lm_head */
        } else {
            j->N = a == 0 ? QD + 2 * KVD : a == 3 ? 2 * MOE * U : a == 4 ? H * U : shapes[a][0];
            j->K = shapes[a][1];
        }
        if (j->N > maxn) maxn = j->N;
        const size_t nb = x100_tile_bytes(int4, j->N, j->K);
        j->off = *pool_off;
        *pool_off = (*pool_off + 1000003) % POOL;
        hip_ok(hipMalloc(&j->w, nb), "hipMalloc");
        fill(j->w, nb, j->off, st->s);
        st->bytes += nb;
    }
    hip_ok(hipMalloc((void **)&st->dx, (size_t)M * XK), "hipMalloc");
    hip_ok(hipMalloc((void **)&st->dy, (size_t)M * maxn * 4), "hipMalloc");
    hip_ok(hipMemcpyAsync(st->dx, x, (size_t)M * XK, hipMemcpyHostToDevice, st->s), "copy x");
    hip_ok(hipStreamSynchronize(st->s), "sync");
}

static void stream_free(Stream *st)
{
    for (int i = 0; i < st->njobs; i++) hip_ok(hipFree(st->jobs[i].w), "hipFree");
    hip_ok(hipFree(st->dx), "hipFree");
    hip_ok(hipFree(st->dy), "hipFree");
    if (st->exec) hip_ok(hipGraphExecDestroy(st->exec), "hipGraphExecDestroy");
    hip_ok(hipStreamDestroy(st->s), "hipStreamDestroy");
    free(st->jobs);
}

/* ms per token: the token's launches captured once, replayed reps times between two events. */
static double ms_per_token(Stream *st, int reps)
{
    hipGraph_t g;
    for (int i = 0; i < st->njobs; i++) launch(st, &st->jobs[i]);   /* warm-up */
    hip_ok(hipStreamSynchronize(st->s), "sync");
    hip_ok(hipStreamBeginCapture(st->s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    for (int i = 0; i < st->njobs; i++) launch(st, &st->jobs[i]);
    hip_ok(hipStreamEndCapture(st->s, &g), "hipStreamEndCapture");
    hip_ok(hipGraphInstantiate(&st->exec, g, NULL, NULL, 0), "hipGraphInstantiate");
    hip_ok(hipGraphDestroy(g), "hipGraphDestroy");
    hip_ok(hipGraphLaunch(st->exec, st->s), "hipGraphLaunch");
    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");
    hip_ok(hipEventRecord(e0, st->s), "hipEventRecord");
    for (int r = 0; r < reps; r++) hip_ok(hipGraphLaunch(st->exec, st->s), "hipGraphLaunch");
    hip_ok(hipEventRecord(e1, st->s), "hipEventRecord");
    hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0;
    hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    hip_ok(hipEventDestroy(e0), "hipEventDestroy");
    hip_ok(hipEventDestroy(e1), "hipEventDestroy");
    return ms / reps;
}

/* Every launch once, eagerly, each output compared with the host matmul. */
static int check_stream(Stream *st, const int8_t *x, const char *name)
{
    int bad = 0;
    for (int i = 0; i < st->njobs; i++) {
        char what[96];
        snprintf(what, sizeof what, "%s M=%d U=%d launch %d", name, st->M, st->U, i);
        launch(st, &st->jobs[i]);
        bad |= check_job(st, &st->jobs[i], x, what);
    }
    return bad;
}

int main(int argc, char **argv)
{
    int L = 48, reps = 3, check = 0, json = 0, nus = 0, us[16];
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--layers") && i + 1 < argc) L = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--reps") && i + 1 < argc) reps = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--check")) check = 1;
        else if (!strcmp(argv[i], "--json")) json = 1;
        else if (!strcmp(argv[i], "--us") && i + 1 < argc) {
            for (char *t = strtok(argv[++i], ","); t && nus < 16; t = strtok(NULL, ",")) us[nus++] = atoi(t);
        } else if (argv[i][0] == '-') {
            fprintf(stderr, "usage: moe_decode [nt] [--layers L] [--reps R] [--us 8,16,24,64] [--check] [--json]\n");
            return 2;
        }   /* a bare number is the reference's thread count: ignored */
    }
    if (!nus) us[0] = 8, us[1] = 16, us[2] = 24, us[3] = 64, nus = 4;
    if (L < 1 || reps < 1) return 2;
    x100_hip_caps_t caps;
    x100_ok(x100_hip_detect(&caps), "x100_hip_detect");

    uint8_t *pool = (uint8_t *)malloc(POOL);
    uint64_t seed = 1234;
    for (size_t i = 0; i < POOL / 8; i++) ((uint64_t *)pool)[i] = splitmix64(&seed);
    void *dpool = NULL;
    hip_ok(hipMalloc(&dpool, POOL), "hipMalloc");
    hip_ok(hipMemcpy(dpool, pool, POOL, hipMemcpyHostToDevice), "copy pool");
    g_pool_host = pool, g_pool_dev = (const uint8_t *)dpool;
    int8_t *x = (int8_t *)malloc((size_t)8 * XK);
    for (int i = 0; i < 8 * XK; i++) x[i] = (int8_t)(splitmix64(&seed) & 0xff);

    printf("Qwen3-30B-A3B  H=%d heads=%d/%d hd=%d experts=%d/%d moe_inter=%d L=%d vocab=%d  on %s\n", H, NH, NKV, HD,
           N_EXP, N_ACT, MOE, L, VOCAB, caps.name);
    int bad = 0;
    size_t off = 0;
    char js[4096];
    int jl = snprintf(js, sizeof js, "{\"layers\": %d", L);
    for (int q4 = 1; q4 >= 0; q4--) {
        const char *nm = q4 ? "q4-interlaced" : "q8";
        Stream st;
        stream_init(&st, q4, 1, N_ACT, L, x, &off);
        if (check) bad |= check_stream(&st, x, nm);
        const double ms1 = ms_per_token(&st, reps);
        if (check) bad |= check_job(&st, &st.jobs[st.njobs - 1], x, "graph replay, lm_head");
        const double params = (double)((QD + 2 * KVD) * H + H * QD + N_EXP * H) * L + 3.0 * MOE * H * N_ACT * L +
                              (double)VOCAB * H;
        printf("\n[%s]  active params/tok = %.2fB of 30B  (%.0f MB %s/tok)\n", nm, params / 1e9, st.bytes / 1e6, nm);
        printf("  M=1 single-stream : %.3f ms/tok -> %.1f tok/s   (%.1f GB/s)\n", ms1, 1e3 / ms1, st.bytes / ms1 / 1e6);
        jl += snprintf(js + jl, sizeof js - jl, ", \"%s\": {\"bytes_per_token\": %zu, \"m1_ms_per_token\": %.5f, "
                       "\"m1_tok_s\": %.2f, \"m1_GB_s\": %.1f", q4 ? "q4" : "q8", st.bytes, ms1, 1e3 / ms1,
                       st.bytes / ms1 / 1e6);
        stream_free(&st);
        printf("  M=8 MTP verify (8 tokens/pass), by expert-union U:\n");
        for (int ui = 0; ui < nus; ui++) {
            const int U = us[ui] > N_EXP ? N_EXP : us[ui];
            stream_init(&st, q4, 8, U, L, x, &off);
            if (check) bad |= check_stream(&st, x, nm);
            const double msU = ms_per_token(&st, reps);
            if (check) bad |= check_job(&st, &st.jobs[st.njobs - 1], x, "graph replay, lm_head");
            const double tps = 8.0 / msU * 1e3;
            const char *tag = U == 8 ? "perfect overlap" : U == 64 ? "disjoint (worst)" : "partial overlap";
            printf("     U=%-3d (%-16s): %.3f ms/pass -> %.1f tok/s  (%.1fx vs M=1, %.1f GB/s)\n", U, tag, msU, tps,
                   tps / (1e3 / ms1), st.bytes / msU / 1e6);
            jl += snprintf(js + jl, sizeof js - jl, ", \"m8_u%d_ms_per_pass\": %.5f, \"m8_u%d_tok_s\": %.1f", U, msU, U,
                           tps);
            stream_free(&st);
        }
        jl += snprintf(js + jl, sizeof js - jl, "}");
    }
    if (check) printf("\ncheck: %s\n", bad ? "MISMATCH" : "every launch equals the host matmul");
    if (json) printf("%s, \"check\": %s}\n", js, check ? (bad ? "false" : "true") : "null");
    hip_ok(hipFree(dpool), "hipFree");
    free(pool);
    free(x);
    return bad ? 1 : 0;
}
