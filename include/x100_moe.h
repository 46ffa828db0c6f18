/*
 * x100_moe.h -- Qwen3-MoE decode layer entry point of libx100hip (gfx950).
 *
 * The FFN block of the reference's forward() (qwen_moe.c:294-311; qwen_moe_hp.c:1512-1570) for
 * M token rows (decode, speculative verify or prefill), one call per layer:
 *   logits = R . hn (fp32), softmax over all n_exp experts, top-n_act (ties -> lower expert id),
 *   renormalised weights; for each selected expert: g = Wg[e].hn, u = Wu[e].hn, act = silu(g)*u,
 *   y = Wd[e].act; out = sum_a w_a * y_a  (plus out's old value with X100_MOE_RESIDUAL).
 * Experts are Q4_K blocks in the ggml 3-D layout, experts outermost (qwen_moe.c:220-222):
 *   Wg, Wu: [n_exp][ff][d/256] blocks, Wd: [n_exp][d][ff/256] blocks,
 * or the same bytes regrouped by moe_pack_experts (then X100_MOE_TILED in flags).
 *
 * flags (the `residual` argument): bit 0, X100_MOE_RESIDUAL, adds the result into out (the
 * reference's x += moe(x)); bit 1, X100_MOE_TILED, says that Wg, Wu and Wd were written by
 * moe_pack_experts.  Any other bit is rejected (X100_EINVAL).  The results are the same, bit for
 * bit, in both layouts.
 * Activations are quantized to Q8_K per row (hn before gate/up, act before down) with the
 * scalar path's rounding; rows that pick the same expert share one pass over its weights (up to
 * 8 token rows all rows at once; from 9 rows the (row, slot) pairs are grouped by expert into
 * chunks of 32 on the matrix cores, the MUL_MAT_ID grouping of ime.cpp:667-697).  Each row's
 * result is the same as a one-row call's, bit for bit.
 *
 * All pointers are device pointers.  sel / sw (may be NULL) receive [M][n_act] expert ids and
 * renormalised weights.  Limits: 1 <= M <= X100_MOE_MAX_ROWS, 1 <= n_act <= 8, n_act <= n_exp <= 256,
 * d % 256 == 0, ff % 256 == 0, d <= 4096, ff <= 4096; hn, R, Wg, Wu, Wd 16-byte aligned.
 *
 * Scratch: the reference's linears take caller scratch (the packed activation and partial sums,
 * qwen_moe.c:90-101; per-thread buffers, qwen_moe_hp.c:712-718).  moe_layer_hip_ws does the same:
 * the caller passes a device buffer of moe_layer_workspace_bytes(...) bytes; the call allocates
 * nothing and never synchronises, so it can be captured into a HIP graph at any shape, and calls
 * on different streams run concurrently when their buffers differ.  moe_layer_hip is the
 * convenience form: the library keeps one workspace per (device, stream), grown by hipMalloc when
 * a larger shape arrives (outgrown buffers are kept until the process ends, so graphs captured
 * earlier stay valid); a call that would grow it while its stream is being captured returns
 * X100_EINVAL.  Workspace contents never need initialising.
 */
#ifndef X100_HIP_MOE_H
#define X100_HIP_MOE_H

#include <stddef.h>
#include <stdint.h>

#define X100_MOE_MAX_ROWS 512
#define X100_MOE_RESIDUAL 1   /* flags: out += the layer's result (else out = it)                 */
#define X100_MOE_TILED    2   /* flags: expert tensors in moe_pack_experts' layout               */
/* Size of moe_layer_hip_noalloc's static scratch array (8 MiB per GPU): enough for up to 64
 * token rows at the Qwen3-30B-A3B shape (d 2048, ff 768, 128 experts, top 8) and 16 rows at
 * d = ff = 4096. */
#define X100_MOE_NOALLOC_MAX_BYTES ((size_t)8 << 20)
#define X100_ESCRATCH   -8   /* the shape needs more scratch than X100_MOE_NOALLOC_MAX_BYTES    */

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces the MoE block of forward(), qwen_moe.c:294-311 (and qwen_moe_hp.c:1512-1570). */
int moe_layer_hip(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                  const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                  int *sel, float *sw, void *stream);

/* Device scratch bytes moe_layer_hip_ws needs for this shape; 0 outside the limits above. */
size_t moe_layer_workspace_bytes(int M, int d, int ff, int n_exp, int n_act);

/* moe_layer_hip on caller scratch ws (device, 256-byte aligned, ws_bytes >=
 * moe_layer_workspace_bytes(M, d, ff, n_exp, n_act)), in the way lin_mm takes xt
 * (qwen_moe.c:101).  Calls whose executions overlap must use distinct buffers. */
int moe_layer_hip_ws(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                     const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                     int *sel, float *sw, void *ws, size_t ws_bytes, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): moe_layer_hip with
 * its scratch in a static device array of X100_MOE_NOALLOC_MAX_BYTES per GPU, set up on the first
 * call on each GPU; the call allocates nothing, frees nothing and never synchronises.  A shape
 * whose moe_layer_workspace_bytes exceeds the array returns X100_ESCRATCH with nothing enqueued.
 * All calls on one GPU share the array: calls whose executions overlap on one GPU (other streams,
 * or graphs replayed concurrently) race and must use moe_layer_hip_ws instead.  The array keeps
 * the last call's contents; nothing in it needs clearing between calls. */
int moe_layer_hip_noalloc(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                          const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                          int *sel, float *sw, void *stream);

/* No counterpart in the reference: a load-time step, like x100q_pack for the GEMV weights.  Copies
 * n_exp expert matrices of rows x K Q4_K weights (ggml layout, as above: Wg and Wu with rows = ff,
 * K = d; Wd with rows = d, K = ff) from src to dst (device, 16-byte aligned, not overlapping, the
 * same n_exp * rows * K / 256 * 144 bytes) in the tiled layout that moe_layer_hip* read with
 * X100_MOE_TILED: per 8 rows and super-block, the 16-byte pieces of the 8 blocks grouped by
 * position (the 8 headers, then bytes 0-15 of the 8 rows' qs, ...), so that the matrix-core path
 * (9 or more token rows) reads whole cache lines.  rows % 8 == 0, K % 256 == 0.  Asynchronous on
 * stream. */
int moe_pack_experts(int n_exp, int rows, int K, const void *src, void *dst, void *stream);

#ifdef __cplusplus
}
#endif
#endif
