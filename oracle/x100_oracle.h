/*
 * x100_oracle.h -- CPU restatement of the reference's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library (libx100hip.so) links, loads or
 * calls this code.  It is used by tests/ (parity checks), by __graft_entry__.smoke() (one small
 * parity check) and by bench.py's cpu_baseline leg (timed scalar baseline).
 *
 * Every function cites the reference file:line whose algorithm it restates.  Numeric conventions
 * that the reference leaves open (or gets differently in different files) are fixed here and
 * implemented identically by the HIP kernels:
 *   - fp32 -> fp16 is the reference's f32_to_f16 (qwen_moe_hp.c:71-79): the magnitude is
 *     truncated (round toward zero, fp16 subnormals included), |f| >= 2^16 and NaN give a signed
 *     infinity.  Every fp16 scale the reference writes goes through it (quantize_q8_0_native,
 *     quantize_q4_0_native, and lin_new_i8's requantization via quantize_q8_0_native);
 *   - Q8_0 activations: amax floored at 1e-6, d = amax/127, q = rint(x * (1/d)) (half-even,
 *     with the fp32 d), clamp [-128,127], d stored as fp16 (qwen_moe_hp.c:408-414);
 *   - Q8_K activations: amax (no floor), d = amax/127 kept in fp32, q = roundf(x * (1/d))
 *     (half away from zero), clamp [-128,127], all-zero block -> d = 0, q = 0
 *     (qwen_moe_q3k.c:612-624; rvv_kernels.cpp:1820-1828); bsums are the plain (positive)
 *     16-element sums, ggml order {f32 d; i8 qs[256]; i16 bsums[16]};
 *   - SiLU and the router softmax use exp evaluated in binary64 and rounded once to binary32
 *     (the reference's libm expf differs by at most one ulp);
 *   - the router dot products and the softmax sum use one fixed order (64 lane-strided partial
 *     sums, then a butterfly over the partials), the order the HIP kernel uses, so expert choice
 *     and weights match it bit for bit;
 *   - the float combine of a row's per-block integer dots: K-quants sequential in block order
 *     with no fused multiply-add (build with -ffp-contract=off); Q4_0 and the int8 path in the
 *     kernels' lane order (lane-strided partial sums and their DPP prefix-sum reduction), which
 *     differs from the reference's sequential order by rounding only.
 *
 * Parity pinning (what checks each function beyond itself) is listed in the test files
 * tests/test_oracle.py and tests/golden/.
 */
#ifndef X100_ORACLE_H
#define X100_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF / ggml type ids (bench/gguf_dump.c:12-13). */
#define ORC_Q4_0 2
#define ORC_Q8_0 8
#define ORC_Q3_K 11
#define ORC_Q4_K 12
#define ORC_Q5_K 13
#define ORC_Q6_K 14
#define ORC_Q8_K 15

/* fp16 <-> fp32.  f16_to_f32 follows qwen_moe_hp.c:80-86 (exact); f32_to_f16 follows
 * qwen_moe_hp.c:71-79 (truncation, see header note). */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);

/* ---- int8 GEMM ---------------------------------------------------------------------------- */
/* C[MxN] += A[MxK] * B[KxN], row-major, int32 accumulate; i-k-j loop of src/gemm_ref.c:17-26. */
void gemm_ref_i8(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C);
/* Same arithmetic, rows split over nthreads OpenMP threads (for checking large shapes). */
void orc_gemm_i8_mt(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C,
                    int nthreads);

/* ---- integer tile GEMV (bench/q4_gemv.c) --------------------------------------------------- */
/* y[M][N] = W[N][K] . x[M][K]^T, int32 exact: ref_gemv, bench/q4_gemv.c:101-103. */
void orc_gemv_int(int M, int N, int K, const int8_t *W, const int8_t *x, int32_t *y);
/* Packed weight layouts of pack_w_int4 (bench/q4_gemv.c:37-48) and pack_w_int8 (:55-62).
 * Return 0, or -1 for N % 8 / K % 32 (int4) / K % 16 (int8). */
int orc_pack_w_int4(int N, int K, const int8_t *W, uint8_t *Wq);
int orc_pack_w_int8(int N, int K, const int8_t *W, int8_t *Wp);

/* ---- block formats ------------------------------------------------------------------------- */
size_t orc_block_bytes(int qtype);   /* 18, 34, 110, 144, 176, 210, 292 */
int    orc_block_elems(int qtype);   /* 32 or 256 */
size_t orc_row_bytes(int qtype, int K);

/* Dequantize one row of K elements (GGUF-native blocks) to fp32.
 * Q4_0: qwen_moe.c:164-165.  Q4_K: repack.cpp:222-233 + 950-970.  Q3_K: qwen_moe_q3k.c:557-577.
 * Q8_0: qwen_moe.c:162-163.  Q5_K: qwen_moe_q3k.c:540-551.  Q6_K: qwen_moe.c:168-177.
 * Q8_K: value q*d. */
int orc_dequant_row(int qtype, const void *blocks, int K, float *out);

/* Activation quantizers (see header note).  x has K elements; K % 32 (Q8_0) or K % 256 (Q8_K). */
void orc_quantize_q8_0(const float *x, int K, void *out);
void orc_quantize_q8_K(const float *x, int K, void *out);

/* int8-path activation quantizer pack_A_i8 (qwen_moe_q3k.c:420-427): per 32 elements a 38-byte
 * record {f32 scale; i16 sum; i8 qs[32]}, scale = max(amax, 1e-6)/127 kept in fp32, rint. */
void orc_quantize_i8(const float *x, int K, void *out);
/* Load-time requantization of a Q8_0 / Q5_K / Q6_K weight to Q8_0 (lin_new_i8,
 * qwen_moe_q3k.c:872-886): dequantize each row, re-encode per 32 with orc_quantize_q8_0.
 * Wq8 gets N rows of K/32 Q8_0 blocks.  Returns 0, or -1 for another type / shape. */
int orc_requant_q8_0(int qtype, int N, int K, const void *W, void *Wq8);
/* Weight-side Q4_0 encoder (qwen_moe_hp.c:100-109, fp16 rounding per header note). Used by
 * tests to build weights from float matrices. */
void orc_quantize_q4_0(const float *w, int K, void *out);

/* ---- quantized GEMV -------------------------------------------------------------------------
 * y[M][N] = W[N][K] . x[M][K]^T.  W is GGUF-native blocks, row n at n*row_bytes.  Each x row
 * is quantized on its own (Q8_0 for Q4_0 weights, Q8_K for Q4_K/Q3_K, pack_A_i8 records for
 * the int8 path).  Per block the integer dot is exact; the row result is the sequential fp32 sum
 * over blocks of
 *   Q4_0: (dw*dx) * isum                                (ggml vec_dot_q4_0_q8_0 formula)
 *   Q4_K: dx * (d*isum_sc - dmin*isum_m)                (ggml vec_dot_q4_K_q8_K formula)
 *   Q3_K: dx * (d*isum_sc)                              (ggml vec_dot_q3_K_q8_K formula)
 *   Q8_0 / Q5_K / Q6_K: the weight is first requantized to Q8_0 (orc_requant_q8_0), then per
 *     K32 group acc = fma(dw*scale, isum, acc)        (run_i8_m1, qwen_moe_q3k.c:428-510)
 * Returns 0, or -1 for an unsupported type / shape. */
int orc_qgemv(int qtype, int M, int N, int K, const void *W, const float *x, float *y);

/* The per-call part of the int8 path: y = Wq8 . x^T for a weight already requantized by
 * orc_requant_q8_0 (N rows of K/32 Q8_0 blocks); x rows are quantized with orc_quantize_i8. */
int orc_qgemv_q8w(int M, int N, int K, const void *Wq8, const float *x, float *y);
/* Same result from already-quantized activations (xq = M rows of Q8_0 / Q8_K blocks or
 * pack_A_i8 records). */
int orc_qgemv_q(int qtype, int M, int N, int K, const void *W, const void *xq, float *y);

/* ---- MoE decode layer -----------------------------------------------------------------------
 * The FFN block of qwen_moe.c:294-311 for M token rows of already-normalised hidden state hn:
 *   logits = R . hn (fp32), softmax over all n_exp (qwen_moe.c:189), top-n_act by
 *   repeated strict-> argmax (lower index wins ties, :299-300), renormalise (:301), then per
 *   selected expert a = 0..n_act-1:  g = Wg[e].q8k(hn), u = Wu[e].q8k(hn) (Q4_K x Q8_K),
 *   act = silu(g)*u, y = Wd[e].q8k(act), out += w_a * y   (:303-310).
 * Wg, Wu: [n_exp][ff][d/256] Q4_K blocks;  Wd: [n_exp][d][ff/256] Q4_K blocks (ggml 3-D layout,
 * experts outermost, qwen_moe.c:220-222).  out[M][d] is overwritten (residual add = flag).
 * sel/sw (optional, may be NULL) receive [M][n_act] expert ids and renormalised weights.
 * d % 256 == 0, n_exp <= 256.  Returns 0 or -1 on bad shapes. */
int orc_moe_layer(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                  const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                  int *sel, float *sw);

/* Router stage only: logits (pre-softmax) [M][n_exp], sel, sw.  Used to report top-k margins. */
int orc_moe_route(int M, int d, int n_exp, int n_act, const float *hn, const float *R,
                  float *logits, int *sel, float *sw);

/* SiLU-gated product used by the MoE block (qwen_moe.c:309 / qwen_moe_hp.c:1307-1309). */
float orc_swiglu(float g, float u);

/* ---- decode step around the MoE block -------------------------------------------------------- */
/* rmsnorm (qwen_moe.c:187), rope table and rotation (qwen_moe_hp.c:799-804; pow/cos/sin in
 * binary64, rounded once). */
void orc_rmsnorm(float *o, const float *x, const float *w, int n, float eps);
void orc_rope_table(float *cosb, float *sinb, int hd, int pos, float base);
void orc_rope_apply(float *v, int hd, const float *cosb, const float *sinb);

typedef struct {
    int d, n_head, n_head_kv, head_dim, ff, n_exp, n_act, ctx;
    float eps, rope_base;
    int wq_type, wk_type, wv_type, wo_type;   /* ggml type ids of the attention weights */
} orc_layer_cfg;

/* Attention half of a decoder layer for one token (qwen_moe.c:279-293): h += Wo.attn(...), and
 * k, v written at pos of the head-major caches kc, vc [n_head_kv][ctx][head_dim].  Weights are
 * GGUF-native blocks, row-major (Wq: n_head*head_dim rows of d; Wk, Wv: n_head_kv*head_dim rows
 * of d; Wo: d rows of n_head*head_dim).  Returns 0 or -1. */
int orc_attn_decode(const orc_layer_cfg *c, const float *attn_norm, const float *q_norm, const float *k_norm,
                    const void *wq, const void *wk, const void *wv, const void *wo, float *kc, float *vc, int pos,
                    float *h);
/* Whole layer (qwen_moe.c:278-311): attention half, rmsnorm(ffn_norm), h += MoE (orc_moe_layer). */
int orc_decode_layer(const orc_layer_cfg *c, const float *attn_norm, const float *q_norm, const float *k_norm,
                     const void *wq, const void *wk, const void *wv, const void *wo, const float *ffn_norm,
                     const float *router, const void *wg, const void *wu, const void *wd, float *kc, float *vc,
                     int pos, float *h, int *sel, float *sw);

#ifdef __cplusplus
}
#endif
#endif
