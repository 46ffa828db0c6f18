/*
 * Driver for the reference's own scalar format functions (test infrastructure, never the product).
 *
 * oracle/ref_scalar.py copies the named definitions out of the reference's qwen_moe_q3k.c into a
 * temporary file REF_SCALAR_SRC and compiles this driver with it into oracle/_ref/libref_scalar.so
 * (and libref_scalar_fma.so, the same with a*b - c contracted into FMAs).
 * The functions are `static` in the reference, so the driver includes their text and exports thin
 * wrappers with plain pointer/size arguments for ctypes:
 *
 *   ref_f32_to_f16      f32_to_f16            qwen_moe_q3k.c:71-79  (truncating fp32 -> fp16)
 *   ref_f16_to_f32      f16_to_f32            qwen_moe_q3k.c:80-86
 *   ref_f16f            f16f                  qwen_moe_q3k.c:1089-1092 (the loader's fp16 -> fp32)
 *   ref_q8_0            quantize_q8_0_native  qwen_moe_q3k.c:409-414  (34-byte blocks)
 *   ref_pack_a_i8       pack_A_i8             qwen_moe_q3k.c:420-427  (38-byte records)
 *   ref_pack_a_q3k      pack_A_q3k            qwen_moe_q3k.c:613-623  (292-byte Q8_K records)
 *   ref_dequant         gguf_dequant_into     qwen_moe_q3k.c:1129-1158 (Q4_0, Q8_0, Q3_K, Q5_K, Q6_K;
 *                       Q3_K and Q5_K through dequantize_q3_K_block / dequantize_q5_K_block,
 *                       :557-577 / :540-551)
 *   ref_requant_q8_0    lin_new_i8's per-row algorithm (:872-886): gguf_dequant_into of the row,
 *                       then quantize_q8_0_native per 32 elements
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include REF_SCALAR_SRC

#define EXPORT __attribute__((visibility("default")))

EXPORT void ref_f32_to_f16(const float *x, size_t n, uint16_t *out)
{
    for (size_t i = 0; i < n; i++) out[i] = f32_to_f16(x[i]);
}

EXPORT void ref_f16_to_f32(const uint16_t *h, size_t n, float *out)
{
    for (size_t i = 0; i < n; i++) out[i] = f16_to_f32(h[i]);
}

EXPORT void ref_f16f(const uint16_t *h, size_t n, float *out)
{
    for (size_t i = 0; i < n; i++) out[i] = f16f(h[i]);
}

EXPORT void ref_q8_0(const float *x, size_t ngroups, uint8_t *out)
{
    for (size_t g = 0; g < ngroups; g++) {
        q8_0_native b;
        quantize_q8_0_native(x + 32 * g, &b);
        memcpy(out + 34 * g, &b.d, 2);
        memcpy(out + 34 * g + 2, b.qs, 32);
    }
}

EXPORT void ref_pack_a_i8(const float *x, size_t ngroups, uint8_t *out)
{
    for (size_t g = 0; g < ngroups; g++) pack_A_i8(x + 32 * g, out + 38 * g);
}

EXPORT void ref_pack_a_q3k(const float *x, size_t nsb, uint8_t *out)
{
    for (size_t s = 0; s < nsb; s++) pack_A_q3k(x + 256 * s, out + 292 * s);
}

/* n elements of GGUF type typ from blocks (a whole number of blocks).  Returns 0, or -1 for a type
 * the reference's loader does not take. */
EXPORT int ref_dequant(uint32_t typ, const uint8_t *blocks, size_t n, float *out)
{
    if (typ != 2 && typ != 8 && typ != 11 && typ != 13 && typ != 14) return -1;
    Gguf g;
    TInfo ti;
    memset(&g, 0, sizeof g);
    memset(&ti, 0, sizeof ti);
    g.p = (unsigned char *)blocks;
    g.data_start = 0;
    ti.typ = typ;
    ti.off = 0;
    gguf_dequant_into(&g, &ti, 0, n, out);
    return 0;
}

/* rows x K elements of GGUF type typ (row r's blocks at r * row_bytes) -> rows x K/32 34-byte Q8_0
 * blocks, as lin_new_i8 computes them before packing its records. */
EXPORT int ref_requant_q8_0(uint32_t typ, const uint8_t *w, size_t rows, size_t K, size_t row_bytes, uint8_t *out)
{
    float *tmp = (float *)malloc(K * sizeof(float));
    if (!tmp) return -1;
    for (size_t r = 0; r < rows; r++) {
        if (ref_dequant(typ, w + r * row_bytes, K, tmp)) {
            free(tmp);
            return -1;
        }
        ref_q8_0(tmp, K / 32, out + r * (K / 32) * 34);
    }
    free(tmp);
    return 0;
}
