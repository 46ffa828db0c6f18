// Internal launch interfaces between the C-ABI layer (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "x100_decode.h"
#include "x100_moe.h"

enum {
    X100_GEMM_AUTO = 0,
    X100_GEMM_TILE256 = 1,
    X100_GEMM_TILE128 = 2,
    X100_GEMM_SKINNY = 3,
    X100_GEMM_GENERIC = 4,
    X100_GEMM_TILE256_W4 = 5,   // 256x256 tile, 4 waves of 128x128
    X100_GEMM_TILE64 = 6,       // 64x64 tile, 4 waves of 32x32
    X100_GEMM_TILE32 = 7,       // 32x32 tile, 1 wave
};

// acc: C += A.B; otherwise the overwrite form C = A.B.
hipError_t x100_gemm_i8_launch(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C,
                               hipStream_t s, int variant, bool acc);
hipError_t x100_zero_i32_launch(int32_t *C, size_t n, hipStream_t s);

size_t x100_q_packed_bytes(int qtype, int N, int K);
hipError_t x100_q_pack_launch(int qtype, int N, int K, const void *src, void *dst, hipStream_t s);
hipError_t x100_qgemv_launch(int qtype, int M, int N, int K, const void *w, const float *x, float *y,
                             hipStream_t s);
// Two one-row GEMVs of one weight type on the same x (packed weights w0: N0 x K, w1: N1 x K) in one
// launch, each row's result that of x100_qgemv_launch; hipErrorNotSupported (nothing launched)
// for shapes or types that have no merged form.
hipError_t x100_qgemv2_launch(int qtype, int N0, const void *w0, float *y0, int N1, const void *w1, float *y1, int K,
                              const float *x, hipStream_t s);
// The same two plus a third one-row GEMV on the int8 path (qtype2: Q8_0, Q5_K or Q6_K, packed
// w2: N2 x K) in one launch; hipErrorNotSupported (nothing launched) outside the shapes it has.
// With nrm, x is a raw row and the products take RMSNorm(x) with weights nrm and eps (the
// operations of the norm launch it replaces, bit for bit).
hipError_t x100_qgemv3_launch(int qtype, int N0, const void *w0, float *y0, int N1, const void *w1, float *y1,
                              int qtype2, int N2, const void *w2, float *y2, int K, const float *x, const float *nrm,
                              float eps, hipStream_t s);
// True when x100_qgemv_launch accepts the shape (it then launches without further checks).
bool x100_qgemv_supported(int qtype, int M, int N, int K);
hipError_t x100_check_quant_div_launch(uint32_t lo, uint32_t hi, unsigned long long *cnt, hipStream_t s);

size_t x100_moe_workspace_bytes(int M, int d, int ff, int n_exp, int n_act);
// flags: X100_MOE_RESIDUAL, X100_MOE_TILED (x100_moe.h).
hipError_t x100_moe_launch(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                           const void *Wg, const void *Wu, const void *Wd, float *out, int flags,
                           int *sel, float *sw, void *workspace, hipStream_t s);
hipError_t x100_moe_tile_pack(int n_exp, int rows, int K, const void *src, void *dst, hipStream_t s);
// One token row of a decoder layer with the step before the MoE block folded in: h <- (h + o) +
// MoE(rmsnorm(h + o, nrm)), the bits of h += o, hn = rmsnorm(h, nrm), x100_moe_launch(hn, out = h,
// residual).  Supported (x100_moe_norm_supported) for d = 2048, flags X100_MOE_RESIDUAL (ggml-layout
// experts, as the decoder layer keeps them).
bool x100_moe_norm_supported(int d, int ff, int n_exp, int n_act, int flags);
hipError_t x100_moe_norm_launch(int d, int ff, int n_exp, int n_act, float *h, const float *o, const float *nrm,
                                float eps, const float *R, const void *Wg, const void *Wu, const void *Wd, int flags,
                                int *sel, float *sw, void *workspace, hipStream_t s);

hipError_t x100_gemv_tile_launch(int int4, int M, int N, int K, const void *W, const int8_t *x, int32_t *y,
                                 hipStream_t s);

// Attention half of a decoder layer (attn.hip).  ws holds x100_attn_workspace_bytes(c) bytes; with
// w->ffn_norm set, *hn_out receives rmsnorm(h, ffn_norm) (inside ws) for the MoE block.  With
// o_out, h += o and the norm are left to the caller (x100_moe_norm_launch): *o_out receives o.
size_t x100_attn_workspace_bytes(const x100_layer_cfg *c);
hipError_t x100_attn_launch(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h,
                            float *ws, float **hn_out, hipStream_t s, float **o_out = nullptr);

