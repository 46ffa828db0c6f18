// The decode step around the MoE block, for one token (qwen_moe.c:278-293): RMSNorm, the q / k / v
// GEMVs (qgemv.hip), per-head RMSNorm + RoPE with the KV-cache write, grouped-query attention split
// over position chunks (flash-decoding) and merged, the output GEMV and the residual add.
//
// Launches for the attention half: rmsnorm, 3 GEMVs, qk_rope, attn_part, attn_combine, 1 GEMV,
// residual (+ the next rmsnorm, fused).  The work between the GEMVs is small (a few KB per head);
// the attention reads each KV-cache row once per block (K and V: 1 KiB per position and KV head).
#include <float.h>

#include <algorithm>

#include <cmath>

#include "x100_common.h"
#include "x100_internal.h"

namespace {

constexpr int HD = 128;   // head_dim of the kernels below (Qwen3)

// RMSNorm of one row (qwen_moe.c:187): s = 1/sqrt(mean(x^2) + eps), out = (x*s)*w.  One block.  With
// add != NULL the residual x += add is done first and written back (qwen_moe.c:293, fused with the
// norm that follows it); with w == NULL only the residual is done.
template <int NT>
__global__ __launch_bounds__(NT) void k_rmsnorm(float *__restrict__ x, const float *__restrict__ add,
                                                const float *__restrict__ w, float eps, int n,
                                                float *__restrict__ out)
{
    __shared__ float red[NT / 64];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += NT) {
        float v = x[i];
        if (add) {
            v += add[i];
            x[i] = v;
        }
        ss += v * v;
    }
    if (!w) return;
    ss = wave_sum_bfly_f(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < NT / 64; k++) tot += red[k];
    const float s = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += NT) out[i] = x[i] * s * w[i];
}

// e^x evaluated in double and rounded once (the oracle does the same; libm's expf differs by at most
// one ulp).
X100_DEV float exp_r(float x) { return (float)exp((double)x); }

// 8-lane all-reduce (lanes 8g .. 8g+7): xor 1, xor 2 within quads, then the half-row mirror pairs
// each lane with one of the other quad.
X100_DEV float sum8_all(float v)
{
    v += dpp_f<0xB1>(0.0f, v);
    v += dpp_f<0x4E>(0.0f, v);
    v += dpp_f<0x141>(0.0f, v);
    return v;
}

// Attention over one chunk of positions for one KV head (qwen_moe.c:289-292: scores q.K_j/sqrt(hd),
// softmax over j, o = sum_j p_j V_j).  Block (kvh, c) covers positions [c*CH, min((c+1)*CH, n_pos))
// for the gpr query heads of KV head kvh; wave w takes the heads w, w+4, ... (QPW of them).  A wave
// steps through the chunk 8 positions at a time: 8 lanes per position, each with 16 of the 128
// dimensions of K_j and V_j, keeping a running maximum m, sum l and output o per position group and
// head (online softmax).  The 8 groups are then merged, and lanes 0-7 write (m, l, o[128]) of each
// head to part[head][c].
// The rotation of the token's position for every pair (i, i + HD/2), passed by value in the kernel
// arguments: the launcher builds it on the host once per call, as the reference builds its rope
// table there (qwen_moe_hp.c:799-804).
struct RopeTab {
    float cs[HD / 2], sn[HD / 2];
};

template <int QPW>
__global__ __launch_bounds__(256) void k_attn_part(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, const float *__restrict__ q_norm,
                                                   const float *__restrict__ k_norm, float eps, const RopeTab rt,
                                                   float *__restrict__ kc, float *__restrict__ vc, int gpr, int ctx,
                                                   int n_pos, int CH, float scale, float *__restrict__ part)
{
    constexpr int DL = HD / 8;
    __shared__ float s_q[4 * QPW][HD];   // the block's query heads after RMSNorm and RoPE
    const int kvh = blockIdx.x, c = blockIdx.y, nch = gridDim.y, pos = n_pos - 1;
    const int lane = threadIdx.x & 63, w = wave_id(), grp = lane >> 3, sl = lane & 7;
    const int j0 = c * CH, j1 = min(j0 + CH, n_pos);
    const bool has_pos = c == nch - 1;   // the chunk holding pos writes this KV head's cache rows
    const float *K = kc + (size_t)kvh * ctx * HD + sl * DL, *V = vc + (size_t)kvh * ctx * HD + sl * DL;

    // The K / V rows of the next step are loaded before the current step is computed.
    float kr[DL], vr[DL], kn[DL], vn[DL];
    auto load_rows = [&](int jb, float (&kk)[DL], float (&vv)[DL]) {
        const int j = jb + grp;
        const size_t row = (size_t)(j < j1 ? j : j0) * HD;
#pragma unroll
        for (int t = 0; t < DL; t += 4) {
            const float4 a = *(const float4 *)(K + row + t), b4 = *(const float4 *)(V + row + t);
            kk[t] = a.x; kk[t + 1] = a.y; kk[t + 2] = a.z; kk[t + 3] = a.w;
            vv[t] = b4.x; vv[t + 1] = b4.y; vv[t + 2] = b4.z; vv[t + 3] = b4.w;
        }
    };
    if (!has_pos) load_rows(j0, kr, vr);   // rows written before this launch: load at once

    // Per-head RMSNorm and RoPE (qwen_moe.c:284-285; rope table qwen_moe_hp.c:799-804): lane i
    // rotates the pair (i, i + HD/2) by the table's cos and sin.  Wave w takes the block's query heads w, w+4, ... (clamped: heads past gpr repeat the
    // last and are not stored); in the chunk holding pos, wave 0 also writes this KV head's key row
    // (normalised and rotated) and value row into the cache at pos and waits for the stores, which
    // the barrier below orders before every wave's loads of that row.
    {
        const int i = lane;
        const float cs = rt.cs[i], sn = rt.sn[i];
        auto norm_rope = [&](const float *src, const float *wn, float &o0, float &o1) {
            const float x = src[i], y = src[i + HD / 2];
            const float ss = wave_sum_bfly_f(x * x + y * y);
            const float s = 1.0f / sqrtf(ss / (float)HD + eps);
            const float a0 = x * s * wn[i], a1 = y * s * wn[i + HD / 2];
            o0 = a0 * cs - a1 * sn;
            o1 = a0 * sn + a1 * cs;
        };
#pragma unroll
        for (int g = 0; g < QPW; g++) {
            const int hq = w + 4 * g;
            float o0, o1;
            norm_rope(q + ((size_t)kvh * gpr + min(hq, gpr - 1)) * HD, q_norm, o0, o1);
            s_q[hq][i] = o0;
            s_q[hq][i + HD / 2] = o1;
        }
        if (has_pos && w == 0) {
            float o0, o1;
            norm_rope(k + (size_t)kvh * HD, k_norm, o0, o1);
            float *kd = kc + ((size_t)kvh * ctx + pos) * HD, *vd = vc + ((size_t)kvh * ctx + pos) * HD;
            kd[i] = o0;
            kd[i + HD / 2] = o1;
            vd[i] = v[(size_t)kvh * HD + i];
            vd[i + HD / 2] = v[(size_t)kvh * HD + i + HD / 2];
            __builtin_amdgcn_s_waitcnt(0);   // the cache row is in memory before the barrier
        }
    }
    __syncthreads();
    if (has_pos) load_rows(j0, kr, vr);

    float qr[QPW][DL], m[QPW], l[QPW], o[QPW][DL];
#pragma unroll
    for (int g = 0; g < QPW; g++) {
#pragma unroll
        for (int t = 0; t < DL; t++) qr[g][t] = s_q[w + 4 * g][sl * DL + t];
        m[g] = -FLT_MAX;
        l[g] = 0.0f;
#pragma unroll
        for (int t = 0; t < DL; t++) o[g][t] = 0.0f;
    }
    for (int jb = j0; jb < j1; jb += 8) {
        const bool more = jb + 8 < j1;
        if (more) load_rows(jb + 8, kn, vn);
        const bool ok = jb + grp < j1;
#pragma unroll
        for (int g = 0; g < QPW; g++) {
            float d = 0.0f;
#pragma unroll
            for (int t = 0; t < DL; t++) d = __builtin_fmaf(qr[g][t], kr[t], d);
            const float sc = sum8_all(d) * scale;
            // m' = max(m, sc): one of e^(m - m') and e^(sc - m') is e^0 = 1, so one exp suffices
            const bool up = ok && sc > m[g];
            const float ex = exp_r(up ? m[g] - sc : sc - m[g]);
            const float corr = up ? ex : 1.0f;
            const float p = ok ? (up ? 1.0f : ex) : 0.0f;
            l[g] = l[g] * corr + p;
#pragma unroll
            for (int t = 0; t < DL; t++) o[g][t] = __builtin_fmaf(o[g][t], corr, p * vr[t]);
            m[g] = up ? sc : m[g];
        }
        if (more) {
#pragma unroll
            for (int t = 0; t < DL; t++) {
                kr[t] = kn[t];
                vr[t] = vn[t];
            }
        }
    }

    // merge the 8 position groups (lanes l, l^8, l^16, l^32 hold the same dimensions): xor 8 is a
    // rotation by 8 within a row of 16 (DPP), xor 16 and xor 32 are permlane swaps
#pragma unroll
    for (int g = 0; g < QPW; g++) {
#pragma unroll
        for (int lvl = 0; lvl < 3; lvl++) {
            auto xch = [&](float v) { return lvl == 0 ? dpp_f<0x128>(v, v) : (lvl == 1 ? xor16_f(v) : xor32_f(v)); };
            const float m2 = xch(m[g]), l2 = xch(l[g]);
            // a = e^(m - max), b = e^(m2 - max): one of them is 1
            const bool mine = m[g] >= m2;
            const float ex = exp_r(mine ? m2 - m[g] : m[g] - m2);
            const float a = mine ? 1.0f : ex, b = mine ? ex : 1.0f;
            l[g] = l[g] * a + l2 * b;
#pragma unroll
            for (int t = 0; t < DL; t++) o[g][t] = o[g][t] * a + xch(o[g][t]) * b;
            m[g] = mine ? m[g] : m2;
        }
        const int hq = w + 4 * g;
        if (hq < gpr && grp == 0) {
            // per head: m[nch], l[nch], then o[nch][HD] (a chunk's 128 dimensions contiguous, so the
            // combine reads each chunk with whole-line loads)
            float *P = part + (size_t)(kvh * gpr + hq) * nch * (HD + 2);
            if (sl == 0) {
                P[c] = m[g];
                P[nch + c] = l[g];
            }
            float *Pc = P + 2 * (size_t)nch + (size_t)c * HD + sl * DL;   // 4-byte aligned only
#pragma unroll
            for (int t = 0; t < DL; t++) Pc[t] = o[g][t];
        }
    }
}

// Merge the chunks of one query head: att = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M).  The
// maximum M (exact in any order) and the weights e_c are computed once per chunk, spread over the
// threads, into LDS; the two sums then run in chunk order in every thread (the order the oracle
// uses), thread t reading dimension t of each chunk (one contiguous 512-byte row per chunk for
// the block).  nch <= 512.
__global__ __launch_bounds__(HD) void k_attn_combine(const float *__restrict__ part, int nch, float *__restrict__ att)
{
    __shared__ float se[512], red[HD / 64];
    const int h = blockIdx.x, t = threadIdx.x;
    const float *P = part + (size_t)h * nch * (HD + 2);
    float mx = -FLT_MAX;
    for (int c = t; c < nch; c += HD) {
        se[c] = P[c];
        mx = fmaxf(mx, se[c]);
    }
    mx = fmaxf(mx, xor32_f(mx));
    mx = fmaxf(mx, xor16_f(mx));
    mx = fmaxf(mx, dpp_f<0x128>(mx, mx));
    mx = fmaxf(mx, dpp_f<0x124>(mx, mx));
    mx = fmaxf(mx, dpp_f<0x4E>(mx, mx));
    mx = fmaxf(mx, dpp_f<0xB1>(mx, mx));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int k = 1; k < HD / 64; k++) M = fmaxf(M, red[k]);
    for (int c = t; c < nch; c += HD) se[c] = exp_r(se[c] - M);
    __syncthreads();
    const float *Lc = P + nch, *Oc = P + 2 * (size_t)nch + t;
    float L = 0.0f, O = 0.0f;
#pragma unroll 16
    for (int c = 0; c < nch; c++) {
        const float e = se[c];
        L += Lc[c] * e;
        O += Oc[(size_t)c * HD] * e;
    }
    att[(size_t)h * HD + t] = O / L;
}

// Chunking of 0..pos: about 256 blocks over the KV heads, at least 8 positions per chunk (512
// blocks made each block's fixed cost, the merge and the partial stores, and the combine's chunk
// loop weigh more: a Qwen3 layer took 51.0 / 54.2 us at 1024 / 4096 positions against 48.1 /
// 52.9 us; 128 blocks: 48.5 / 58.4 us).  Since CH >= n_pos / target and CH >= 8,
// nch <= min(target, ceil(n_pos / 8)) for every n_pos.
int chunk_target(int n_kv) { return n_kv >= 256 ? 1 : 256 / n_kv; }
void chunks(int n_pos, int n_kv, int &CH, int &nch)
{
    const int target = chunk_target(n_kv);
    CH = (n_pos + target - 1) / target;
    CH = (CH + 7) / 8 * 8;
    if (CH < 8) CH = 8;
    nch = (n_pos + CH - 1) / CH;
}

constexpr size_t seg(size_t floats) { return (floats + 63) / 64 * 64; }   // 256-byte segments

// fr = base^(-2i/hd) with the exponent in fp32, a = pos*fr in fp32, as the reference; pow, cos and
// sin evaluated in double and rounded once (the oracle's orc_rope_table).
RopeTab rope_table(int pos, float base)
{
    RopeTab t;
    for (int i = 0; i < HD / 2; i++) {
        const float e = -2.0f * (float)i / (float)HD;
        const float fr = (float)std::pow((double)base, (double)e);
        const float a = (float)pos * fr;
        t.cs[i] = (float)std::cos((double)a);
        t.sn[i] = (float)std::sin((double)a);
    }
    return t;
}

}  // namespace

// Workspace floats: hn[d] q[qd] k[kvd] v[kvd] att[qd] o[d] part[n_head][nch_max][HD + 2].
size_t x100_attn_workspace_bytes(const x100_layer_cfg *c)
{
    const int nch = std::min(chunk_target(c->n_head_kv), (c->ctx + 7) / 8);   // bound for every pos < ctx
    const size_t qd = (size_t)c->n_head * HD, kvd = (size_t)c->n_head_kv * HD;
    return 4 * (seg(c->d) * 2 + seg(qd) * 2 + seg(kvd) * 2 + seg((size_t)c->n_head * nch * (HD + 2)));
}

hipError_t x100_attn_launch(const x100_layer_cfg *c, const x100_layer_weights *w, int pos, float *h,
                            float *ws, float **hn_out, hipStream_t s, float **o_out)
{
    const int d = c->d, nh = c->n_head, nkv = c->n_head_kv, gpr = nh / nkv, qd = nh * HD, kvd = nkv * HD;
    float *hn = ws, *q = hn + seg(d), *k = q + seg(qd), *v = k + seg(kvd), *att = v + seg(kvd),
          *o = att + seg(qd), *part = o + seg(d);
    hipError_t e;
    // q, v and k in one launch when q and v share a K-quant type and k is on the int8 path (Q3_K
    // and Q8_0 in the mixed checkpoint, d = 2048), with the attention RMSNorm of h inside it (its
    // 16-byte loads of h and the norm weights need both 16-byte aligned); else
    // the norm launch, then q and v in one launch when they share a weight type that has the
    // merged form, else one launch each
    e = c->wq_type == c->wv_type && w->attn_norm && !(((uintptr_t)h | (uintptr_t)w->attn_norm) & 15)
            ? x100_qgemv3_launch(c->wq_type, qd, w->wq, q, kvd, w->wv, v, c->wk_type, kvd, w->wk, k, d, h,
                                 w->attn_norm, c->eps, s)
            : hipErrorNotSupported;
    if (e != hipSuccess && e != hipErrorNotSupported) return e;
    const bool qvk = e == hipSuccess;
    if (!qvk)
        hipLaunchKernelGGL(k_rmsnorm<1024>, dim3(1), dim3(1024), 0, s, h, (const float *)nullptr, w->attn_norm,
                           c->eps, d, hn);
    e = !qvk && c->wq_type == c->wv_type ? x100_qgemv2_launch(c->wq_type, qd, w->wq, q, kvd, w->wv, v, d, hn, s)
                                         : hipErrorNotSupported;
    if (e != hipSuccess && e != hipErrorNotSupported) return e;
    const bool qv = qvk || e == hipSuccess;
    if (!qv && (e = x100_qgemv_launch(c->wq_type, 1, qd, d, w->wq, hn, q, s)) != hipSuccess) return e;
    if (!qvk && (e = x100_qgemv_launch(c->wk_type, 1, kvd, d, w->wk, hn, k, s)) != hipSuccess) return e;
    if (!qv && (e = x100_qgemv_launch(c->wv_type, 1, kvd, d, w->wv, hn, v, s)) != hipSuccess) return e;
    // head norms, RoPE and the KV-cache write at pos run inside the attention blocks (k_attn_part)
    int CH, nch;
    chunks(pos + 1, nkv, CH, nch);
    const float scale = 1.0f / sqrtf((float)HD);
    const RopeTab rt = rope_table(pos, c->rope_base);
    const dim3 grid(nkv, nch);
#define X100_ATTN(QPW)                                                                                  \
    hipLaunchKernelGGL(k_attn_part<QPW>, grid, dim3(256), 0, s, q, k, v, w->q_norm, w->k_norm, c->eps, rt, \
                       w->k_cache, w->v_cache, gpr, c->ctx, pos + 1, CH, scale, part)
    if (gpr <= 4)
        X100_ATTN(1);
    else if (gpr <= 8)
        X100_ATTN(2);
    else
        X100_ATTN(4);
#undef X100_ATTN
    hipLaunchKernelGGL(k_attn_combine, dim3(nh), dim3(HD), 0, s, part, nch, att);
    if ((e = x100_qgemv_launch(c->wo_type, 1, d, qd, w->wo, att, o, s)) != hipSuccess) return e;
    if (o_out) {   // the caller's MoE launch adds o and forms the norm itself
        *o_out = o;
        return hipGetLastError();
    }
    // h += o, and hn = rmsnorm(h, ffn_norm) for the MoE block that follows (skipped without ffn_norm)
    hipLaunchKernelGGL(k_rmsnorm<1024>, dim3(1), dim3(1024), 0, s, h, (const float *)o, w->ffn_norm, c->eps, d, hn);
    if (hn_out) *hn_out = hn;
    return hipGetLastError();
}
