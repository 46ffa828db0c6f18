/*
 * x100_decode.h -- one Qwen3-MoE decoder layer for one token, device-resident (libx100hip, gfx950).
 *
 * Replaces the per-layer body of the reference's forward() (qwen_moe.c:278-311; the same steps in
 * qwen_moe_hp.c:1444-1570):
 *   hn = rmsnorm(h, attn_norm); q, k, v = Wq.hn, Wk.hn, Wv.hn;
 *   per head rmsnorm(q_norm / k_norm) + rope(pos); k, v stored at pos of the KV cache;
 *   grouped-query attention over positions 0..pos; h += Wo.att;
 *   hn = rmsnorm(h, ffn_norm); h += MoE(hn)                          (x100_decode_layer_hip only)
 * The GEMVs are qgemv_hip on weights packed by x100q_pack (any of its types); the MoE block is
 * moe_layer_hip on the Q4_K expert tensors.  Numerics follow the reference step by step in fp32
 * (rope's pow / cos / sin and the softmax's exp are evaluated accurately; the attention softmax is
 * computed over position chunks and merged, equal to the sequential one within rounding).
 *
 * All pointers are device pointers; the caches are head-major [n_head_kv][ctx][head_dim] fp32
 * (the layout of qwen_moe_hp.c:1469-1474).  Asynchronous on stream.  Every argument is checked
 * before any work is enqueued: an error return leaves h and the caches as they were.
 *
 * Scratch: the _ws forms take a caller device buffer (256-byte aligned) of at least
 * x100_decode_workspace_bytes(cfg) bytes (the reference's forward takes its scratch vectors hn, q,
 * k, v, att, tmp, g, u, eout, xt from the caller, qwen_moe.c:272-273), allocate nothing and never
 * synchronise, so a captured graph can hold them; overlapping calls need distinct buffers.  The plain forms use the
 * library's per-(device, stream) workspace, as moe_layer_hip does (x100_moe.h).
 */
#ifndef X100_HIP_DECODE_H
#define X100_HIP_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int d;              /* hidden size (embedding_length)                                       */
    int n_head;         /* query heads                                                          */
    int n_head_kv;      /* key/value heads (n_head % n_head_kv == 0, at most 16 query heads each) */
    int head_dim;       /* 128                                                                  */
    int ff;             /* expert feed-forward size (expert_feed_forward_length)                */
    int n_exp, n_act;   /* experts, experts used per token                                      */
    int ctx;            /* KV-cache capacity in positions                                       */
    float eps;          /* rms-norm epsilon                                                     */
    float rope_base;    /* rope.freq_base                                                       */
    int wq_type, wk_type, wv_type, wo_type;   /* ggml type ids of the packed attention weights  */
} x100_layer_cfg;

typedef struct {
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm;   /* [d], [head_dim], [head_dim], [d]      */
    const void *wq, *wk, *wv, *wo;     /* x100q_pack output: Wq n_head*head_dim x d, Wk / Wv
                                          n_head_kv*head_dim x d, Wo d x n_head*head_dim          */
    const float *router;               /* [n_exp][d]                                            */
    const void *wg, *wu, *wd;          /* Q4_K expert tensors as in moe_layer_hip                */
    float *k_cache, *v_cache;          /* [n_head_kv][ctx][head_dim]                            */
} x100_layer_weights;

/* The attention half: h[d] += Wo.attention(...), and k, v written at pos of the caches.
 * 0 <= pos < ctx.  Returns X100_OK or X100_EINVAL / X100_E*. */
int x100_attn_decode_hip(const x100_layer_cfg *cfg, const x100_layer_weights *w, int pos, float *h,
                         void *stream);

/* The whole layer: the attention half, then h += MoE(rmsnorm(h, ffn_norm)).  sel / sw (device,
 * n_act entries each, may be NULL) receive the chosen experts and their weights. */
int x100_decode_layer_hip(const x100_layer_cfg *cfg, const x100_layer_weights *w, int pos, float *h,
                          int *sel, float *sw, void *stream);

/* Scratch bytes of the _ws forms for this configuration (the attention half's share, plus the
 * MoE block's when cfg's n_exp / n_act / ff describe one); 0 for an invalid configuration. */
size_t x100_decode_workspace_bytes(const x100_layer_cfg *cfg);

/* x100_attn_decode_hip / x100_decode_layer_hip on caller scratch ws of ws_bytes bytes. */
int x100_attn_decode_hip_ws(const x100_layer_cfg *cfg, const x100_layer_weights *w, int pos, float *h,
                            void *ws, size_t ws_bytes, void *stream);
int x100_decode_layer_hip_ws(const x100_layer_cfg *cfg, const x100_layer_weights *w, int pos, float *h,
                             int *sel, float *sw, void *ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
