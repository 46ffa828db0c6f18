/*
 * x100_oracle.c -- CPU restatement of the reference's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY (see x100_oracle.h).  Built with -ffp-contract=off so that every
 * fp32 expression rounds after each operation, exactly as written.
 */
#include "x100_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------
 * fp16 helpers
 * ------------------------------------------------------------------------------------------- */

/* fp32 -> fp16 as the reference's f32_to_f16 (qwen_moe_hp.c:71-79) converts: the fp16 exponent is
 * the fp32 one rebiased; a normal result keeps the top 10 mantissa bits (the other 13 are
 * dropped, never rounded up); below the fp16 normal range the mantissa with its leading one is
 * shifted into the subnormal field (again dropping bits), and below 2^-24 the result is a signed
 * zero; an exponent past the fp16 range (|f| >= 2^16, inf, NaN) gives a signed infinity.  For
 * |f| < 2^16 this is round-toward-zero.  Checked in tests/test_oracle.py against an independent
 * round-toward-zero restatement and hand-computed cases. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e16 = (int)((x >> 23) & 0xffu) - 127 + 15;
    const uint32_t frac = x & 0x7fffffu;
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e16 > 0) return (uint16_t)(sign | ((uint32_t)e16 << 10) | (frac >> 13));
    if (e16 < -10) return (uint16_t)sign;
    return (uint16_t)(sign | ((frac | 0x800000u) >> (14 - e16)));
}

/* Exact fp16 -> fp32; same decoding as f16_to_f32 in qwen_moe_hp.c:80-86 and f16f in
 * qwen_moe.c:115-118. */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { e++; mant <<= 1; } while (!(mant & 0x400u));
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15u + 127u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ---------------------------------------------------------------------------------------------
 * int8 GEMM
 * ------------------------------------------------------------------------------------------- */

/* src/gemm_ref.c:17-26: i-k-j order, C += A*B, int32 accumulate. */
void gemm_ref_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C)
{
    for (int i = 0; i < M; i++)
        for (int k = 0; k < K; k++) {
            int32_t a = A[(size_t)i * K + k];
            const int8_t *b = &B[(size_t)k * N];
            int32_t *c = &C[(size_t)i * N];
            for (int j = 0; j < N; j++) c[j] += a * (int32_t)b[j];
        }
}

void orc_gemm_i8_mt(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C,
                    int nthreads)
{
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int i = 0; i < M; i++)
        for (int k = 0; k < K; k++) {
            int32_t a = A[(size_t)i * K + k];
            const int8_t *b = &B[(size_t)k * N];
            int32_t *c = &C[(size_t)i * N];
            for (int j = 0; j < N; j++) c[j] += a * (int32_t)b[j];
        }
}

/* ---- integer tile GEMV ---------------------------------------------------------------------- */

/* bench/q4_gemv.c:101-103: plain dot per (m, n). */
void orc_gemv_int(int M, int N, int K, const int8_t *W, const int8_t *x, int32_t *y)
{
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            int32_t a = 0;
            for (int k = 0; k < K; k++) a += (int32_t)W[(size_t)n * K + k] * (int32_t)x[(size_t)m * K + k];
            y[(size_t)m * N + n] = a;
        }
}

/* bench/q4_gemv.c:37-48: tile (nb, kp) of 128 bytes; byte 16n+k holds W[8nb+n][32kp+k] in the low
 * nibble and W[8nb+n][32kp+16+k] in the high nibble. */
int orc_pack_w_int4(int N, int K, const int8_t *W, uint8_t *Wq)
{
    if (N % 8 || K % 32) return -1;
    const int nkp = K / 32;
    for (int nb = 0; nb < N / 8; nb++)
        for (int kp = 0; kp < nkp; kp++)
            for (int j = 0; j < 128; j++) {
                const int n = j / 16, k = j % 16;
                const int8_t lo = W[(size_t)(8 * nb + n) * K + 32 * kp + k];
                const int8_t hi = W[(size_t)(8 * nb + n) * K + 32 * kp + 16 + k];
                Wq[((size_t)nb * nkp + kp) * 128 + j] = (uint8_t)((lo & 0xf) | ((hi & 0xf) << 4));
            }
    return 0;
}

/* bench/q4_gemv.c:55-62: tile (nb, kb) of 128 bytes; byte 16n+k = W[8nb+n][16kb+k]. */
int orc_pack_w_int8(int N, int K, const int8_t *W, int8_t *Wp)
{
    if (N % 8 || K % 16) return -1;
    const int nkb = K / 16;
    for (int nb = 0; nb < N / 8; nb++)
        for (int kb = 0; kb < nkb; kb++)
            for (int j = 0; j < 128; j++)
                Wp[((size_t)nb * nkb + kb) * 128 + j] = W[(size_t)(8 * nb + j / 16) * K + 16 * kb + j % 16];
    return 0;
}

/* ---------------------------------------------------------------------------------------------
 * Block formats (Appendix of the block-format layouts used by ggml; reference restatements at
 * qwen_moe_hp.c:98, qwen_moe_q3k.c:531, repack.cpp:222-233)
 * ------------------------------------------------------------------------------------------- */

typedef struct { uint16_t d; uint8_t qs[16]; } orc_q4_0;                       /*  18 B */
typedef struct { uint16_t d; int8_t qs[32]; } orc_q8_0;                        /*  34 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } orc_q4_K; /* 144 B */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } orc_q3_K; /* 110 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } orc_q8_K;        /* 292 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } orc_q5_K; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } orc_q6_K;  /* 210 B */
/* pack_A_i8 record (qwen_moe_q3k.c:420-427): fp32 scale, int16 sum, 32 int8, 38 B unpadded. */
typedef struct __attribute__((packed)) { float s; int16_t asum; int8_t qs[32]; } orc_a_i8;

size_t orc_block_bytes(int qtype)
{
    switch (qtype) {
    case ORC_Q4_0: return sizeof(orc_q4_0);
    case ORC_Q8_0: return sizeof(orc_q8_0);
    case ORC_Q4_K: return sizeof(orc_q4_K);
    case ORC_Q3_K: return sizeof(orc_q3_K);
    case ORC_Q8_K: return sizeof(orc_q8_K);
    case ORC_Q5_K: return sizeof(orc_q5_K);
    case ORC_Q6_K: return sizeof(orc_q6_K);
    default: return 0;
    }
}

int orc_block_elems(int qtype)
{
    switch (qtype) {
    case ORC_Q4_0: case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q3_K: case ORC_Q8_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return 0;
    }
}

size_t orc_row_bytes(int qtype, int K)
{
    int qk = orc_block_elems(qtype);
    if (qk == 0 || K % qk) return 0;
    return (size_t)(K / qk) * orc_block_bytes(qtype);
}

/* get_scale_min_k4 (repack.cpp:222-233; same unpack as q5k_get_scale_min, qwen_moe_q3k.c:534-537). */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q3_K 6-bit scale unpack exactly as dequantize_q3_K_block does it (qwen_moe_q3k.c:559-563):
 * bytes 0..11 viewed as three little-endian u32, low nibbles + 2-bit high parts. */
static void q3k_scales(const uint8_t *s12, int8_t out[16])
{
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    memcpy(aux, s12, 12);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    memcpy(out, aux, 16);
}

/* Q3_K element value index helpers (qwen_moe_q3k.c:565-575): element e = 128*h + 32*j + l
 * (h in 0..1, j in 0..3, l in 0..31) takes bits (2j, 2j+1) of qs[32h + l], the high bit from
 * hmask[l] bit (4h + j) (set -> +0, clear -> -4), and sub-block scale index 8h + 2j + l/16. */
static int q3k_value(const orc_q3_K *b, int e)
{
    int h = e >> 7, j = (e >> 5) & 3, l = e & 31;
    int lo = (b->qs[32 * h + l] >> (2 * j)) & 3;
    int hb = (b->hmask[l] >> (4 * h + j)) & 1;
    return lo - (hb ? 0 : 4);
}

int orc_dequant_row(int qtype, const void *blocks, int K, float *out)
{
    int qk = orc_block_elems(qtype);
    if (qk == 0 || K % qk) return -1;
    int nb = K / qk;
    switch (qtype) {
    case ORC_Q4_0: {                                   /* qwen_moe.c:164-165 */
        const orc_q4_0 *b = (const orc_q4_0 *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            float d = orc_f16_to_f32(b[ib].d);
            for (int j = 0; j < 32; j++) {
                int nib = (j < 16) ? (b[ib].qs[j] & 0xf) : (b[ib].qs[j - 16] >> 4);
                out[ib * 32 + j] = (float)(nib - 8) * d;
            }
        }
        return 0;
    }
    case ORC_Q8_0: {                                   /* qwen_moe.c:162-163 */
        const orc_q8_0 *b = (const orc_q8_0 *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            float d = orc_f16_to_f32(b[ib].d);
            for (int j = 0; j < 32; j++) out[ib * 32 + j] = (float)b[ib].qs[j] * d;
        }
        return 0;
    }
    case ORC_Q4_K: {                                   /* repack.cpp:950-970 decode */
        const orc_q4_K *b = (const orc_q4_K *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            float d = orc_f16_to_f32(b[ib].d), dmin = orc_f16_to_f32(b[ib].dmin);
            for (int j = 0; j < 8; j++) {
                int sc, m;
                scale_min_k4(j, b[ib].scales, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                const uint8_t *q = b[ib].qs + 32 * (j / 2);
                for (int l = 0; l < 32; l++) {
                    int nib = (j & 1) ? (q[l] >> 4) : (q[l] & 0xf);
                    out[ib * 256 + 32 * j + l] = d1 * (float)nib - m1;
                }
            }
        }
        return 0;
    }
    case ORC_Q3_K: {                                   /* qwen_moe_q3k.c:557-577 */
        const orc_q3_K *b = (const orc_q3_K *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            int8_t sc[16];
            q3k_scales(b[ib].scales, sc);
            float dall = orc_f16_to_f32(b[ib].d);
            for (int e = 0; e < 256; e++) {
                int is = 8 * (e >> 7) + 2 * ((e >> 5) & 3) + ((e & 31) >> 4);
                float dl = dall * (float)(sc[is] - 32);
                out[ib * 256 + e] = dl * (float)q3k_value(&b[ib], e);
            }
        }
        return 0;
    }
    case ORC_Q5_K: {                                   /* qwen_moe_q3k.c:540-551 */
        const orc_q5_K *b = (const orc_q5_K *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            float d = orc_f16_to_f32(b[ib].d), dmin = orc_f16_to_f32(b[ib].dmin);
            /* 64-element chunk c: sub-blocks 2c (low nibbles, qh bit 2c) and 2c+1 (high
             * nibbles, qh bit 2c+1) of qs[32c .. 32c+31] */
            for (int c = 0; c < 4; c++) {
                for (int hi = 0; hi < 2; hi++) {
                    int sc, m;
                    scale_min_k4(2 * c + hi, b[ib].scales, &sc, &m);
                    float d1 = d * (float)sc, m1 = dmin * (float)m;
                    for (int l = 0; l < 32; l++) {
                        int q = hi ? (b[ib].qs[32 * c + l] >> 4) : (b[ib].qs[32 * c + l] & 0xf);
                        if ((b[ib].qh[l] >> (2 * c + hi)) & 1) q += 16;
                        out[ib * 256 + 64 * c + 32 * hi + l] = d1 * (float)q - m1;
                    }
                }
            }
        }
        return 0;
    }
    case ORC_Q6_K: {                                   /* qwen_moe.c:168-177 */
        const orc_q6_K *b = (const orc_q6_K *)blocks;
        for (int ib = 0; ib < nb; ib++) {
            float d = orc_f16_to_f32(b[ib].d);
            for (int h = 0; h < 2; h++) {
                const uint8_t *ql = b[ib].ql + 64 * h, *qh = b[ib].qh + 32 * h;
                const int8_t *sc = b[ib].scales + 8 * h;
                float *o = out + ib * 256 + 128 * h;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    o[l] = d * (float)sc[is] * (float)q1;
                    o[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    o[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    o[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
        return 0;
    }
    case ORC_Q8_K: {
        const orc_q8_K *b = (const orc_q8_K *)blocks;
        for (int ib = 0; ib < nb; ib++)
            for (int j = 0; j < 256; j++) out[ib * 256 + j] = (float)b[ib].qs[j] * b[ib].d;
        return 0;
    }
    }
    return -1;
}

/* ---------------------------------------------------------------------------------------------
 * Quantizers
 * ------------------------------------------------------------------------------------------- */

/* quantize_q8_0_native, qwen_moe_hp.c:408-414 (fp16 d by the truncating f32_to_f16). */
void orc_quantize_q8_0(const float *x, int K, void *out)
{
    orc_q8_0 *b = (orc_q8_0 *)out;
    for (int ib = 0; ib < K / 32; ib++) {
        const float *w = x + (size_t)ib * 32;
        float amax = 1e-6f;
        for (int i = 0; i < 32; i++) {
            float v = fabsf(w[i]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float inv = d ? 1.0f / d : 0.0f;
        b[ib].d = orc_f32_to_f16(d);
        for (int i = 0; i < 32; i++) {
            int q = (int)rintf(w[i] * inv);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            b[ib].qs[i] = (int8_t)q;
        }
    }
}

/* pack_A_q3k, qwen_moe_q3k.c:612-624 (fp32 scale amax/127, roundf, clamp, 16-element sums),
 * all-zero block as rvv_kernels.cpp:1820-1828.  Stored in ggml order with positive sums. */
void orc_quantize_q8_K(const float *x, int K, void *out)
{
    orc_q8_K *b = (orc_q8_K *)out;
    for (int ib = 0; ib < K / 256; ib++) {
        const float *a = x + (size_t)ib * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) {
            float v = fabsf(a[i]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float rep = d ? 1.0f / d : 0.0f;
        b[ib].d = d;
        for (int g = 0; g < 16; g++) {
            int sum = 0;
            for (int l = 0; l < 16; l++) {
                int q = (int)roundf(a[g * 16 + l] * rep);
                if (q > 127) q = 127;
                if (q < -128) q = -128;
                b[ib].qs[g * 16 + l] = (int8_t)q;
                sum += q;
            }
            b[ib].bsums[g] = (int16_t)sum;
        }
    }
}

/* pack_A_i8, qwen_moe_q3k.c:420-427, over K/32 groups (pack_act_i8, :887-889): per 32 elements
 * amax floored at 1e-6, fp32 scale amax/127, q = rint(x * (1/scale)) clamped to [-128,127], and
 * the int16 sum of the 32 q values. */
void orc_quantize_i8(const float *x, int K, void *out)
{
    orc_a_i8 *b = (orc_a_i8 *)out;
    for (int ib = 0; ib < K / 32; ib++) {
        const float *a = x + (size_t)ib * 32;
        float amax = 1e-6f;
        for (int i = 0; i < 32; i++) {
            float v = fabsf(a[i]);
            if (v > amax) amax = v;
        }
        float scale = amax / 127.0f;
        float inv = scale ? 1.0f / scale : 0.0f;
        int sum = 0;
        orc_a_i8 r;
        for (int i = 0; i < 32; i++) {
            int q = (int)rintf(a[i] * inv);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            r.qs[i] = (int8_t)q;
            sum += q;
        }
        r.s = scale;
        r.asum = (int16_t)sum;
        memcpy(&b[ib], &r, sizeof r);
    }
}

/* lin_new_i8 (qwen_moe_q3k.c:872-886) without its 32-row panel interleave: every row of a Q8_0,
 * Q5_K or Q6_K weight is dequantized to fp32 (gguf_dequant_into, qwen_moe_q3k.c:1129-1158) and
 * re-encoded per 32 elements by quantize_q8_0_native (:409-414), as the loader does for attn_k,
 * attn_output and lm_head (:1747-1768).  Wq8 receives N rows of K/32 Q8_0 blocks. */
int orc_requant_q8_0(int qtype, int N, int K, const void *W, void *Wq8)
{
    if (qtype != ORC_Q8_0 && qtype != ORC_Q5_K && qtype != ORC_Q6_K) return -1;
    size_t rb = orc_row_bytes(qtype, K);
    if (!rb || N < 0) return -1;
    float *row = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!row) return -1;
    for (int n = 0; n < N; n++) {
        orc_dequant_row(qtype, (const uint8_t *)W + (size_t)n * rb, K, row);
        orc_quantize_q8_0(row, K, (uint8_t *)Wq8 + (size_t)n * (K / 32) * sizeof(orc_q8_0));
    }
    free(row);
    return 0;
}

/* quantize_q4_0_native, qwen_moe_hp.c:100-109 (fp16 d by the truncating f32_to_f16). */
void orc_quantize_q4_0(const float *w, int K, void *out)
{
    orc_q4_0 *b = (orc_q4_0 *)out;
    for (int ib = 0; ib < K / 32; ib++) {
        const float *x = w + (size_t)ib * 32;
        float amax = 1e-6f;
        for (int i = 0; i < 32; i++) {
            float v = fabsf(x[i]);
            if (v > amax) amax = v;
        }
        float d = amax / 8.0f;
        float inv = d ? 1.0f / d : 0.0f;
        int8_t q[32];
        for (int i = 0; i < 32; i++) {
            int v = (int)rintf(x[i] * inv);
            if (v > 7) v = 7;
            if (v < -8) v = -8;
            q[i] = (int8_t)v;
        }
        b[ib].d = orc_f32_to_f16(d);
        for (int l = 0; l < 16; l++) {
            uint8_t lo = (uint8_t)(q[l] + 8), hi = (uint8_t)(q[l + 16] + 8);
            b[ib].qs[l] = (uint8_t)((lo & 0xf) | ((hi & 0xf) << 4));
        }
    }
}

/* ---------------------------------------------------------------------------------------------
 * Quantized GEMV (integer dot per block, sequential fp32 combine per row)
 * ------------------------------------------------------------------------------------------- */

/* The kernels' reduction of lpr per-lane partial sums p[0..lpr-1] of one row: an inclusive prefix
 * sum in each row of 16 lanes (row_shr 1, 2, 4, 8, with 0 shifted in), then row_bcast 15 into rows
 * 1 and 3 and row_bcast 31 into rows 2 and 3; the row's value is the one left in the last lane.
 * With row sums s0..s3 that is s0 (lpr 16), s1 + s0 (lpr 32), (s3 + s2) + (s1 + s0) (lpr 64). */
static float row_scan16(const float *v)
{
    float a[16], b[16];
    memcpy(a, v, sizeof a);
    for (int k = 1; k < 16; k <<= 1) {
        for (int i = 0; i < 16; i++) b[i] = a[i] + (i >= k ? a[i - k] : 0.0f);
        memcpy(a, b, sizeof a);
    }
    return a[15];
}

static float lane_reduce(const float *p, int lpr)
{
    const float s0 = row_scan16(p);
    if (lpr == 16) return s0;
    const float s1 = row_scan16(p + 16);
    if (lpr == 32) return s1 + s0;
    const float s2 = row_scan16(p + 32) + 0.0f, s3 = row_scan16(p + 48);
    return (s3 + s2) + (s1 + s0);
}

/* Q4_0 x Q8_0 row dot: ggml vec_dot_q4_0_q8_0 formula; nibble order of qwen_moe.c:165.  The float
 * combine follows the kernel: block b goes to lane b % 64, which adds (float)isum * (dw*dx) in
 * block order, and the 64 lane sums are reduced by lane_reduce. */
static float dot_q4_0_q8_0(const orc_q4_0 *w, const orc_q8_0 *x, int nb)
{
    float acc[64];
    for (int l = 0; l < 64; l++) acc[l] = 0.0f;
    for (int ib = 0; ib < nb; ib++) {
        int isum = 0;
        for (int j = 0; j < 16; j++) {
            isum += ((w[ib].qs[j] & 0xf) - 8) * x[ib].qs[j];
            isum += ((w[ib].qs[j] >> 4) - 8) * x[ib].qs[j + 16];
        }
        float dd = orc_f16_to_f32(w[ib].d) * orc_f16_to_f32(x[ib].d);
        acc[ib % 64] = acc[ib % 64] + (float)isum * dd;
    }
    return lane_reduce(acc, 64);
}

/* Q4_K x Q8_K row dot: y = sum_sb dx*d*sum_j sc_j*sum_l q*a - dx*dmin*sum_j m_j*(a-sum of j). */
static float dot_q4_K_q8_K(const orc_q4_K *w, const orc_q8_K *x, int nb)
{
    float acc = 0.0f;
    for (int ib = 0; ib < nb; ib++) {
        int isc = 0, imn = 0;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, w[ib].scales, &sc, &m);
            const uint8_t *q = w[ib].qs + 32 * (j / 2);
            int dot = 0;
            for (int l = 0; l < 32; l++) {
                int nib = (j & 1) ? (q[l] >> 4) : (q[l] & 0xf);
                dot += nib * x[ib].qs[32 * j + l];
            }
            isc += sc * dot;
            imn += m * (x[ib].bsums[2 * j] + x[ib].bsums[2 * j + 1]);
        }
        float dd = x[ib].d * orc_f16_to_f32(w[ib].d);
        float dm = x[ib].d * orc_f16_to_f32(w[ib].dmin);
        acc = acc + (dd * (float)isc - dm * (float)imn);
    }
    return acc;
}

/* Q3_K x Q8_K row dot: y = sum_sb dx*d*sum_is (s_is-32)*sum_16 q3*a (decode of
 * qwen_moe_q3k.c:557-577; exact integer form of gemm_kernel_i8i3k_mrow_ref,
 * ime2_kernels.cpp:127-215, without its fp16 partial sums). */
static float dot_q3_K_q8_K(const orc_q3_K *w, const orc_q8_K *x, int nb)
{
    float acc = 0.0f;
    for (int ib = 0; ib < nb; ib++) {
        int8_t sc[16];
        q3k_scales(w[ib].scales, sc);
        int sub[16] = {0};
        for (int e = 0; e < 256; e++) {
            int is = 8 * (e >> 7) + 2 * ((e >> 5) & 3) + ((e & 31) >> 4);
            sub[is] += q3k_value(&w[ib], e) * x[ib].qs[e];
        }
        int isc = 0;
        for (int is = 0; is < 16; is++) isc += (sc[is] - 32) * sub[is];
        float dd = x[ib].d * orc_f16_to_f32(w[ib].d);
        acc = acc + dd * (float)isc;
    }
    return acc;
}

/* Q8_0 weight x pack_A_i8 activation row dot, run_i8_m1 (qwen_moe_q3k.c:428-510): per K32
 * group the exact int32 dot, then acc += (dw * scale) * float(dot) as one fused multiply-add
 * (vfmul.vf then vfmacc.vv).  The groups are combined in the kernel's order: lpr lanes per row
 * (16 up to K = 2048, 32 up to 4096, 64 beyond), lane j takes groups j, j + lpr, ... in order
 * (bpl of them; a lane past the last group adds fma(0, 0, acc)), and lane_reduce combines them. */
static float dot_q8_0_i8(const orc_q8_0 *w, const orc_a_i8 *x, int nb)
{
    const int lpr = nb <= 64 ? 16 : nb <= 128 ? 32 : 64;
    const int bpl = nb <= 16 ? 1 : nb <= 32 ? 2 : nb <= 256 ? 4 : 8;
    float acc[64];
    for (int l = 0; l < lpr; l++) {
        acc[l] = 0.0f;
        for (int c = 0; c < bpl; c++) {
            const int ib = l + lpr * c;
            if (ib >= nb) {
                acc[l] = fmaf(0.0f, 0.0f, acc[l]);
                continue;
            }
            orc_a_i8 a;
            memcpy(&a, &x[ib], sizeof a);
            int isum = 0;
            for (int j = 0; j < 32; j++) isum += w[ib].qs[j] * a.qs[j];
            float v1 = orc_f16_to_f32(w[ib].d) * a.s;
            acc[l] = fmaf(v1, (float)isum, acc[l]);
        }
    }
    return lane_reduce(acc, lpr);
}

static int is_i8_path(int qtype) { return qtype == ORC_Q8_0 || qtype == ORC_Q5_K || qtype == ORC_Q6_K; }

/* The per-call part of the int8 path: y[M][N] = Wq8 . x^T for a weight already requantized to
 * N rows of K/32 Q8_0 blocks (orc_requant_q8_0): pack_act_i8 of each x row, then run_i8_m1 per
 * row (lin_mm_i8_x, qwen_moe_q3k.c:1075-1081). */
int orc_qgemv_q8w(int M, int N, int K, const void *Wq8, const float *x, float *y)
{
    if (K <= 0 || K % 32 || M < 0 || N < 0) return -1;
    const int nb = K / 32;
    orc_a_i8 *xa = (orc_a_i8 *)malloc(sizeof(orc_a_i8) * (size_t)nb * (size_t)(M > 0 ? M : 1));
    if (!xa) return -1;
    for (int m = 0; m < M; m++) orc_quantize_i8(x + (size_t)m * K, K, xa + (size_t)m * nb);
    const orc_q8_0 *wq = (const orc_q8_0 *)Wq8;
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++)
            y[(size_t)m * N + n] = dot_q8_0_i8(wq + (size_t)n * nb, xa + (size_t)m * nb, nb);
    free(xa);
    return 0;
}

int orc_qgemv_q(int qtype, int M, int N, int K, const void *W, const void *xq, float *y)
{
    if (is_i8_path(qtype)) {
        if (!orc_row_bytes(qtype, K) || K % 32 || M < 0 || N < 0) return -1;
        const int nb = K / 32;
        orc_q8_0 *wq = (orc_q8_0 *)malloc(sizeof(orc_q8_0) * (size_t)nb * (size_t)(N > 0 ? N : 1));
        if (!wq) return -1;
        orc_requant_q8_0(qtype, N, K, W, wq);
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++)
                y[(size_t)m * N + n] = dot_q8_0_i8(wq + (size_t)n * nb, (const orc_a_i8 *)xq + (size_t)m * nb, nb);
        free(wq);
        return 0;
    }
    size_t rb = orc_row_bytes(qtype, K);
    if (!rb || M < 0 || N < 0) return -1;
    int nb = K / orc_block_elems(qtype);
    int xtype = (qtype == ORC_Q4_0) ? ORC_Q8_0 : ORC_Q8_K;
    size_t xrb = orc_row_bytes(xtype, K);
    for (int m = 0; m < M; m++) {
        const uint8_t *xr = (const uint8_t *)xq + (size_t)m * xrb;
        for (int n = 0; n < N; n++) {
            const uint8_t *wr = (const uint8_t *)W + (size_t)n * rb;
            float v;
            if (qtype == ORC_Q4_0)
                v = dot_q4_0_q8_0((const orc_q4_0 *)wr, (const orc_q8_0 *)xr, nb);
            else if (qtype == ORC_Q4_K)
                v = dot_q4_K_q8_K((const orc_q4_K *)wr, (const orc_q8_K *)xr, nb);
            else if (qtype == ORC_Q3_K)
                v = dot_q3_K_q8_K((const orc_q3_K *)wr, (const orc_q8_K *)xr, nb);
            else
                return -1;
            y[(size_t)m * N + n] = v;
        }
    }
    return 0;
}

int orc_qgemv(int qtype, int M, int N, int K, const void *W, const float *x, float *y)
{
    if (is_i8_path(qtype)) {
        if (!orc_row_bytes(qtype, K) || M < 0) return -1;
        orc_a_i8 *xa = (orc_a_i8 *)malloc(sizeof(orc_a_i8) * (size_t)(K / 32) * (size_t)(M > 0 ? M : 1));
        if (!xa) return -1;
        for (int m = 0; m < M; m++) orc_quantize_i8(x + (size_t)m * K, K, xa + (size_t)m * (K / 32));
        int rc = orc_qgemv_q(qtype, M, N, K, W, xa, y);
        free(xa);
        return rc;
    }
    if (qtype != ORC_Q4_0 && qtype != ORC_Q4_K && qtype != ORC_Q3_K) return -1;
    if (!orc_row_bytes(qtype, K)) return -1;
    int xtype = (qtype == ORC_Q4_0) ? ORC_Q8_0 : ORC_Q8_K;
    size_t xrb = orc_row_bytes(xtype, K);
    uint8_t *xq = (uint8_t *)malloc(xrb * (size_t)(M > 0 ? M : 1));
    if (!xq) return -1;
    for (int m = 0; m < M; m++) {
        if (xtype == ORC_Q8_0) orc_quantize_q8_0(x + (size_t)m * K, K, xq + (size_t)m * xrb);
        else orc_quantize_q8_K(x + (size_t)m * K, K, xq + (size_t)m * xrb);
    }
    int rc = orc_qgemv_q(qtype, M, N, K, W, xq, y);
    free(xq);
    return rc;
}

/* ---------------------------------------------------------------------------------------------
 * MoE decode layer
 * ------------------------------------------------------------------------------------------- */

/* Fixed fp32 summation order shared with the HIP kernels: 64 lane-strided partial sums (lane l
 * takes elements 4l..4l+3, then +256, ...) and a butterfly over the 64 partials (pairs l, l^o for
 * o = 32, 16, ..., 1).  The reference sums sequentially (qwen_moe.c:296) or with an RVV reduction
 * (vdot_f32, qwen_moe_hp.c:881-890); the orders differ by rounding only.  n % 256 == 0. */
static float butterfly64(float p[64])
{
    for (int o = 32; o > 0; o >>= 1) {
        float q[64];
        for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ o];
        memcpy(p, q, sizeof q);
    }
    return p[0];
}

static float dot_lane64(const float *a, const float *b, int n)
{
    float p[64];
    for (int l = 0; l < 64; l++) {
        float s = 0.0f;
        for (int k = 4 * l; k < n; k += 256) {
            s += a[k] * b[k];
            s += a[k + 1] * b[k + 1];
            s += a[k + 2] * b[k + 2];
            s += a[k + 3] * b[k + 3];
        }
        p[l] = s;
    }
    return butterfly64(p);
}

/* exp rounded once to binary32 from a binary64 evaluation (the reference calls libm expf; the
 * two differ by at most one binary32 ulp). */
static float exp_f32(float x) { return (float)exp((double)x); }

/* softmax of qwen_moe.c:189: max-subtract, exp, multiply by 1/sum (sum in the order above, with
 * expert e in lane e%64, slot e/64; n <= 256). */
static void softmax_ref(float *x, int n)
{
    float m = -1e30f;
    for (int i = 0; i < n; i++)
        if (x[i] > m) m = x[i];
    float p[64];
    for (int l = 0; l < 64; l++) p[l] = 0.0f;
    for (int i = 0; i < n; i++) x[i] = exp_f32(x[i] - m);
    for (int l = 0; l < 64; l++)
        for (int c = 0; c < 4; c++)
            if (l + 64 * c < n) p[l] += x[l + 64 * c];
    float s = butterfly64(p);
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

float orc_swiglu(float g, float u)
{
    float e = (float)exp(-(double)g);
    return (g / (1.0f + e)) * u;
}

int orc_moe_route(int M, int d, int n_exp, int n_act, const float *hn, const float *R,
                  float *logits, int *sel, float *sw)
{
    if (M < 0 || d <= 0 || d % 256 || n_exp <= 0 || n_exp > 256 || n_act <= 0 || n_act > n_exp) return -1;
    float *p = (float *)malloc(sizeof(float) * (size_t)n_exp);
    if (!p) return -1;
    for (int m = 0; m < M; m++) {
        const float *h = hn + (size_t)m * d;
        for (int e = 0; e < n_exp; e++) {              /* qwen_moe.c:296 */
            float s = dot_lane64(R + (size_t)e * d, h, d);
            p[e] = s;
            if (logits) logits[(size_t)m * n_exp + e] = s;
        }
        softmax_ref(p, n_exp);                        /* qwen_moe.c:298 */
        int *sl = sel + (size_t)m * n_act;
        float *wl = sw + (size_t)m * n_act;
        for (int a = 0; a < n_act; a++) {              /* qwen_moe.c:299-300 */
            int bi = -1;
            float bv = -1;
            for (int e = 0; e < n_exp; e++) {
                int used = 0;
                for (int b = 0; b < a; b++)
                    if (sl[b] == e) used = 1;
                if (!used && p[e] > bv) { bv = p[e]; bi = e; }
            }
            sl[a] = bi;
            wl[a] = bv;
        }
        float ssum = 0;                                /* qwen_moe.c:301 */
        for (int a = 0; a < n_act; a++) ssum += wl[a];
        for (int a = 0; a < n_act; a++) wl[a] /= ssum;
    }
    free(p);
    return 0;
}

int orc_moe_layer(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                  const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                  int *sel, float *sw)
{
    if (M < 0 || d % 256 || ff % 256 || n_act <= 0 || n_act > n_exp || n_act > 64) return -1;
    size_t gu_rb = orc_row_bytes(ORC_Q4_K, d), dn_rb = orc_row_bytes(ORC_Q4_K, ff);
    size_t gu_eb = gu_rb * (size_t)ff, dn_eb = dn_rb * (size_t)d;
    int *sel_l = (int *)malloc(sizeof(int) * (size_t)(M > 0 ? M : 1) * n_act);
    float *sw_l = (float *)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1) * n_act);
    float *g = (float *)malloc(sizeof(float) * (size_t)ff);
    float *u = (float *)malloc(sizeof(float) * (size_t)ff);
    float *y = (float *)malloc(sizeof(float) * (size_t)d);
    float *eout = (float *)malloc(sizeof(float) * (size_t)d);
    orc_q8_K *xq = (orc_q8_K *)malloc(sizeof(orc_q8_K) * (size_t)(d / 256));
    orc_q8_K *aq = (orc_q8_K *)malloc(sizeof(orc_q8_K) * (size_t)(ff / 256));
    int rc = -1;
    if (!sel_l || !sw_l || !g || !u || !y || !eout || !xq || !aq) goto done;
    if (orc_moe_route(M, d, n_exp, n_act, hn, R, NULL, sel_l, sw_l)) goto done;
    for (int m = 0; m < M; m++) {
        const float *h = hn + (size_t)m * d;
        orc_quantize_q8_K(h, d, xq);                   /* activation packed once, qwen_moe.c:303 */
        for (int i = 0; i < d; i++) eout[i] = 0;
        for (int a = 0; a < n_act; a++) {
            int e = sel_l[(size_t)m * n_act + a];
            float w = sw_l[(size_t)m * n_act + a];
            const uint8_t *ge = (const uint8_t *)Wg + (size_t)e * gu_eb;
            const uint8_t *ue = (const uint8_t *)Wu + (size_t)e * gu_eb;
            const uint8_t *de = (const uint8_t *)Wd + (size_t)e * dn_eb;
            for (int i = 0; i < ff; i++) {             /* gate / up, qwen_moe.c:307 */
                g[i] = dot_q4_K_q8_K((const orc_q4_K *)(ge + (size_t)i * gu_rb), xq, d / 256);
                u[i] = dot_q4_K_q8_K((const orc_q4_K *)(ue + (size_t)i * gu_rb), xq, d / 256);
            }
            for (int i = 0; i < ff; i++) g[i] = orc_swiglu(g[i], u[i]);   /* :309 */
            orc_quantize_q8_K(g, ff, aq);
            for (int j = 0; j < d; j++)                /* down + weighted sum, :310 */
                y[j] = dot_q4_K_q8_K((const orc_q4_K *)(de + (size_t)j * dn_rb), aq, ff / 256);
            for (int j = 0; j < d; j++) eout[j] += w * y[j];
        }
        float *o = out + (size_t)m * d;
        for (int j = 0; j < d; j++) o[j] = residual ? o[j] + eout[j] : eout[j];   /* :311 */
    }
    if (sel) memcpy(sel, sel_l, sizeof(int) * (size_t)M * n_act);
    if (sw) memcpy(sw, sw_l, sizeof(float) * (size_t)M * n_act);
    rc = 0;
done:
    free(sel_l); free(sw_l); free(g); free(u); free(y); free(eout); free(xq); free(aq);
    return rc;
}

/* ---------------------------------------------------------------------------------------------
 * Decode step around the MoE block (qwen_moe.c:278-311 with the helpers of :187-189 and the
 * rope table of qwen_moe_hp.c:799-804)
 * ------------------------------------------------------------------------------------------- */

/* rmsnorm, qwen_moe.c:187: s = 1/sqrtf(sum(x^2)/n + eps), o = (x*s)*w.  The sum of squares is
 * taken in the kernel's order: thread t of 1024 sums x_i^2 for i = t, t + 1024, ... in order, each
 * wave of 64 threads combines its sums by the xor butterfly (butterfly64), and the 16 wave sums are
 * added in wave order.  (The reference sums in index order; the two differ by rounding only.) */
void orc_rmsnorm(float *o, const float *x, const float *w, int n, float eps)
{
    float tot = 0.0f;
    for (int wv = 0; wv < 16; wv++) {
        float p[64];
        for (int l = 0; l < 64; l++) {
            float ss = 0.0f;
            for (int i = 64 * wv + l; i < n; i += 1024) ss += x[i] * x[i];
            p[l] = ss;
        }
        tot += butterfly64(p);
    }
    const float s = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * s * w[i];
}

/* The per-head rmsnorm of q and k (qwen_moe.c:284-285) for head_dim 128, in the kernel's order:
 * lane i of 64 holds x_i^2 + x_{i+64}^2, combined by the xor butterfly. */
static void rmsnorm_head128(float *v, const float *w, float eps)
{
    float p[64];
    for (int i = 0; i < 64; i++) p[i] = v[i] * v[i] + v[i + 64] * v[i + 64];
    const float s = 1.0f / sqrtf(butterfly64(p) / 128.0f + eps);
    for (int i = 0; i < 128; i++) v[i] = v[i] * s * w[i];
}

/* rope_table, qwen_moe_hp.c:799-801 (the per-head rope of qwen_moe.c:188 computes the same):
 * fr = base^(-2i/hd) with the exponent in fp32, a = pos*fr in fp32, cos a and sin a.  pow, cos
 * and sin are evaluated in binary64 and rounded once (libm's powf/cosf/sinf differ by an ulp). */
void orc_rope_table(float *cosb, float *sinb, int hd, int pos, float base)
{
    for (int i = 0; i < hd / 2; i++) {
        float e = -2.0f * (float)i / (float)hd;
        float fr = (float)pow((double)base, (double)e);
        float a = (float)pos * fr;
        cosb[i] = (float)cos((double)a);
        sinb[i] = (float)sin((double)a);
    }
}

/* rope_apply, qwen_moe_hp.c:802-804: rotate the pairs (i, i + hd/2). */
void orc_rope_apply(float *v, int hd, const float *cosb, const float *sinb)
{
    for (int i = 0; i < hd / 2; i++) {
        float c = cosb[i], sn = sinb[i], x = v[i], y = v[i + hd / 2];
        v[i] = x * c - y * sn;
        v[i + hd / 2] = x * sn + y * c;
    }
}

static int layer_ok(const orc_layer_cfg *c)
{
    return c && c->d > 0 && c->n_head > 0 && c->n_head_kv > 0 && c->n_head % c->n_head_kv == 0 &&
           c->head_dim == 128 && c->ctx > 0;
}

/* Attention of one query head over positions 0..n_pos-1 of its KV head (K, V: [pos][128]), in the
 * kernels' order (softmax over the scores q.K_j * scale, then o = sum_j p_j V_j):
 *   positions are cut into chunks of CH (attn_chunks); in a chunk, position j belongs to group
 *   (j - j0) % 8, and each group keeps a running maximum m, sum l and output o, updated position by
 *   position (online softmax: corr = e^(m - m'), p = e^(s - m'), l = l*corr + p,
 *   o = fma(o, corr, p*v));
 *   a score is the dot product split in 8 slices of 16 (an fma chain each) summed as
 *   ((d0+d1) + (d2+d3)) + ((d4+d5) + (d6+d7)), times scale;
 *   the 8 groups are merged by the xor butterfly (strides 1, 2, 4), chunk results in chunk order:
 *   att = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).
 * exp is evaluated in binary64 and rounded once.  Equal to the sequential softmax of
 * qwen_moe.c:289-292 up to rounding. */
static void attn_chunks(int n_pos, int n_kv, int *CH, int *nch)
{
    const int target = n_kv >= 256 ? 1 : 256 / n_kv;
    int ch = (n_pos + target - 1) / target;
    ch = (ch + 7) / 8 * 8;
    if (ch < 8) ch = 8;
    *CH = ch;
    *nch = (n_pos + ch - 1) / ch;
}

typedef struct { float m, l, o[128]; } attn_state;

static void attn_merge(attn_state *a, const attn_state *b)
{
    const float mn = fmaxf(a->m, b->m), ea = exp_f32(a->m - mn), eb = exp_f32(b->m - mn);
    a->l = a->l * ea + b->l * eb;
    for (int t = 0; t < 128; t++) a->o[t] = a->o[t] * ea + b->o[t] * eb;
    a->m = mn;
}

static void attn_head(const float *qh, const float *K, const float *V, int n_pos, int n_kv, float scale,
                      float *out)
{
    int CH, nch;
    attn_chunks(n_pos, n_kv, &CH, &nch);
    attn_state *part = (attn_state *)malloc(sizeof(attn_state) * (size_t)nch);
    attn_state g[8], tmp[8];
    for (int c = 0; c < nch; c++) {
        const int j0 = c * CH, j1 = j0 + CH < n_pos ? j0 + CH : n_pos;
        for (int k = 0; k < 8; k++) {
            g[k].m = -FLT_MAX;
            g[k].l = 0.0f;
            for (int t = 0; t < 128; t++) g[k].o[t] = 0.0f;
        }
        for (int jb = j0; jb < j1; jb += 8)
            for (int k = 0; k < 8; k++) {
                const int j = jb + k, ok = j < j1;
                const float *kr = K + (size_t)(ok ? j : j0) * 128, *vr = V + (size_t)(ok ? j : j0) * 128;
                float dl[8];
                for (int sl = 0; sl < 8; sl++) {
                    float dd = 0.0f;
                    for (int t = 0; t < 16; t++) dd = fmaf(qh[16 * sl + t], kr[16 * sl + t], dd);
                    dl[sl] = dd;
                }
                const float sc = (((dl[0] + dl[1]) + (dl[2] + dl[3])) + ((dl[4] + dl[5]) + (dl[6] + dl[7]))) * scale;
                const float mn = ok ? fmaxf(g[k].m, sc) : g[k].m;
                const float corr = exp_f32(g[k].m - mn);
                const float p = ok ? exp_f32(sc - mn) : 0.0f;
                g[k].l = g[k].l * corr + p;
                for (int t = 0; t < 128; t++) g[k].o[t] = fmaf(g[k].o[t], corr, p * vr[t]);
                g[k].m = mn;
            }
        for (int off = 1; off < 8; off <<= 1) {
            for (int k = 0; k < 8; k++) {
                tmp[k] = g[k];
                attn_merge(&tmp[k], &g[k ^ off]);
            }
            memcpy(g, tmp, sizeof g);
        }
        part[c] = g[0];
    }
    float M = -FLT_MAX;
    for (int c = 0; c < nch; c++) M = fmaxf(M, part[c].m);
    float L = 0.0f, O[128];
    for (int t = 0; t < 128; t++) O[t] = 0.0f;
    for (int c = 0; c < nch; c++) {
        const float e = exp_f32(part[c].m - M);
        L += part[c].l * e;
        for (int t = 0; t < 128; t++) O[t] += part[c].o[t] * e;
    }
    for (int t = 0; t < 128; t++) out[t] = O[t] / L;
    free(part);
}

/* Attention half of one decoder layer for one token at position pos (qwen_moe.c:279-293):
 *   hn = rmsnorm(h, attn_norm); q, k, v = Wq.hn, Wk.hn, Wv.hn (quantized GEMVs, orc_qgemv);
 *   per head rmsnorm(q_norm / k_norm) then rope; k, v stored at pos of the head-major caches
 *   kc, vc [n_head_kv][ctx][head_dim] (the layout of qwen_moe_hp.c:1469-1474);
 *   per query head (kv head hh / (n_head / n_head_kv)): scores q.K_j * (1/sqrtf(hd)) for
 *   j = 0..pos, softmax, o = sum_j p_j V_j (attn_head);
 *   h += Wo.att.
 * head_dim 128.  Sums are taken in the kernels' orders (orc_rmsnorm, rmsnorm_head128, attn_head). */
int orc_attn_decode(const orc_layer_cfg *c, const float *attn_norm, const float *q_norm, const float *k_norm,
                    const void *wq, const void *wk, const void *wv, const void *wo, float *kc, float *vc, int pos,
                    float *h)
{
    if (!layer_ok(c) || pos < 0 || pos >= c->ctx) return -1;
    const int d = c->d, nh = c->n_head, nkv = c->n_head_kv, hd = c->head_dim, gpr = nh / nkv;
    const int qd = nh * hd, kvd = nkv * hd;
    float *hn = (float *)malloc(sizeof(float) * (size_t)d), *q = (float *)malloc(sizeof(float) * (size_t)qd);
    float *k = (float *)malloc(sizeof(float) * (size_t)kvd), *v = (float *)malloc(sizeof(float) * (size_t)kvd);
    float *att = (float *)malloc(sizeof(float) * (size_t)qd), *tmp = (float *)malloc(sizeof(float) * (size_t)d);
    float *sc = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
    float *cosb = (float *)malloc(sizeof(float) * (size_t)(hd / 2)), *sinb = (float *)malloc(sizeof(float) * (size_t)(hd / 2));
    int rc = -1;
    if (!hn || !q || !k || !v || !att || !tmp || !sc || !cosb || !sinb) goto done;
    orc_rmsnorm(hn, h, attn_norm, d, c->eps);
    if (orc_qgemv(c->wq_type, 1, qd, d, wq, hn, q) || orc_qgemv(c->wk_type, 1, kvd, d, wk, hn, k) ||
        orc_qgemv(c->wv_type, 1, kvd, d, wv, hn, v))
        goto done;
    orc_rope_table(cosb, sinb, hd, pos, c->rope_base);
    for (int hh = 0; hh < nh; hh++) {
        rmsnorm_head128(q + hh * hd, q_norm, c->eps);
        orc_rope_apply(q + hh * hd, hd, cosb, sinb);
    }
    for (int hh = 0; hh < nkv; hh++) {
        rmsnorm_head128(k + hh * hd, k_norm, c->eps);
        orc_rope_apply(k + hh * hd, hd, cosb, sinb);
        memcpy(kc + ((size_t)hh * c->ctx + pos) * hd, k + hh * hd, sizeof(float) * (size_t)hd);
        memcpy(vc + ((size_t)hh * c->ctx + pos) * hd, v + hh * hd, sizeof(float) * (size_t)hd);
    }
    {
        const float scale = 1.0f / sqrtf((float)hd);
        for (int hh = 0; hh < nh; hh++) {
            const int kvh = hh / gpr;
            attn_head(q + hh * hd, kc + (size_t)kvh * c->ctx * hd, vc + (size_t)kvh * c->ctx * hd, pos + 1, nkv,
                      scale, att + hh * hd);
        }
    }
    if (orc_qgemv(c->wo_type, 1, d, qd, wo, att, tmp)) goto done;
    for (int i = 0; i < d; i++) h[i] += tmp[i];
    rc = 0;
done:
    free(hn); free(q); free(k); free(v); free(att); free(tmp); free(sc); free(cosb); free(sinb);
    return rc;
}

/* One whole decoder layer (qwen_moe.c:278-311): the attention half, then
 * hn = rmsnorm(h, ffn_norm) and h += MoE(hn) (orc_moe_layer with the residual flag). */
int orc_decode_layer(const orc_layer_cfg *c, const float *attn_norm, const float *q_norm, const float *k_norm,
                     const void *wq, const void *wk, const void *wv, const void *wo, const float *ffn_norm,
                     const float *router, const void *wg, const void *wu, const void *wd, float *kc, float *vc,
                     int pos, float *h, int *sel, float *sw)
{
    if (orc_attn_decode(c, attn_norm, q_norm, k_norm, wq, wk, wv, wo, kc, vc, pos, h)) return -1;
    float *hn = (float *)malloc(sizeof(float) * (size_t)c->d);
    if (!hn) return -1;
    orc_rmsnorm(hn, h, ffn_norm, c->d, c->eps);
    int rc = orc_moe_layer(1, c->d, c->ff, c->n_exp, c->n_act, hn, router, wg, wu, wd, h, 1, sel, sw);
    free(hn);
    return rc;
}

