// Qwen3-MoE decode layer (the FFN block of qwen_moe.c:294-311) for M <= 8 token rows.
//
//   k_moe_route    router logits R.hn (one wave per expert), Q8_K of every hn row; the last
//                  block to finish does softmax / top-k / renormalise per row and groups the
//                  (row, slot) pairs by expert (the expert union, as ggml MUL_MAT_ID does,
//                  ime.cpp:667-697).
//   k_moe_gate_up  one block per (selected expert, 8 rows of ff): streams those rows of the
//                  expert's gate and up matrices once for all rows that chose it (Q4_K x Q8_K),
//                  SwiGLU, writes the activation; the last block of an expert quantizes its
//                  activations to Q8_K.
//   k_moe_down     one block per (selected expert, 16 rows of d): down projection of every pair
//                  of that expert; the last block of a row range combines the slots of each token
//                  row in slot order a = 0..n_act-1 (out += w_a * y_a), so results do not depend
//                  on block scheduling.
// Completion is counted with device-scope atomics and fences; no block ever waits for another.
#include "x100_common.h"
#include "x100_internal.h"

namespace {

constexpr int GU_ROWS = 8;    // gate/up rows per block
constexpr int DN_ROWS = 16;   // down rows per block

// Workspace layout (device memory owned by the library, sized by x100_moe_workspace_bytes).
struct MoeWs {
    float *logits;        // [M][n_exp]
    int *sel;             // [M][n_act]
    float *sw;            // [M][n_act]
    int *nuniq;           // [1]
    int *uniq;            // [P]          expert id of union slot u (P = M*n_act)
    int *ucnt;            // [P]          pairs in union slot u
    int *upairs;          // [P][8]       pair ids (m*n_act + a) of union slot u
    int8_t *xq;           // [M][d/256][256]
    int *xbs;             // [M][d/256][16]
    float *xd;            // [M][d/256]
    float *act;           // [P][ff]
    int8_t *aq;           // [P][ff/256][256]
    int *abs_;            // [P][ff/256][16]
    float *ad;            // [P][ff/256]
    float *ydn;           // [P][d]
    int *cnt_route;       // [1]
    int *cnt_gu;          // [P]
    int *cnt_dn;          // [d/DN_ROWS]
};

inline size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

// Quantize one 256-element block to Q8_K with one wave (same operations as pack_A_q3k).
X100_DEV void q8k_block_wave(const float *src, int8_t *qs, int *bs, float *dout)
{
    const int lane = threadIdx.x & 63;
    const float4 v = *(const float4 *)(src + 4 * lane);
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    const float amax = wave_max_f(a);
    const float d = amax / 127.0f;
    const float rep = d != 0.0f ? 1.0f / d : 0.0f;
    const int q0 = clamp_i8((int)roundf(v.x * rep)), q1 = clamp_i8((int)roundf(v.y * rep));
    const int q2 = clamp_i8((int)roundf(v.z * rep)), q3 = clamp_i8((int)roundf(v.w * rep));
    ((uint32_t *)qs)[lane] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                             ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) bs[lane >> 2] = s;
    if (lane == 0) *dout = d;
}

// get_scale_min_k4 (repack.cpp:222-233) over the header dwords 1..3 of a Q4_K block.
X100_DEV uint32_t hbyte(const v4i &h, int k)
{
    const uint32_t w = (uint32_t)(k < 4 ? h[1] : (k < 8 ? h[2] : h[3]));
    return (w >> (8 * (k & 3))) & 0xffu;
}
X100_DEV void gsm(const v4i &h, int j, int &sc, int &m)
{
    if (j < 4) {
        sc = hbyte(h, j) & 63;
        m = hbyte(h, j + 4) & 63;
    } else {
        sc = (hbyte(h, j + 4) & 0xf) | ((hbyte(h, j - 4) >> 6) << 4);
        m = (hbyte(h, j + 4) >> 4) | ((hbyte(h, j) >> 6) << 4);
    }
}

// Integer part of one Q4_K x Q8_K super-block dot over the 8 lanes of a unit (lane i of 8 holds
// qs bytes [16i, 16i+16)).  Returns isc/imn reduced over the 8 lanes.
X100_DEV void q4k_unit_dot(const v4i &hdr, const v4i &qs, const int8_t *xq256, const int *bs16,
                           int i, int &isc, int &imn)
{
    const int p = i >> 1, h = i & 1;
    int sc0, m0, sc1, m1;
    gsm(hdr, 2 * p, sc0, m0);
    gsm(hdr, 2 * p + 1, sc1, m1);
    const v4i xa = *(const v4i *)(xq256 + 64 * p + 16 * h);
    const v4i xc = *(const v4i *)(xq256 + 64 * p + 32 + 16 * h);
    int d0 = 0, d1 = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        d0 = dot4(qs[t] & 0x0F0F0F0F, xa[t], d0);
        d1 = dot4((qs[t] >> 4) & 0x0F0F0F0F, xc[t], d1);
    }
    isc = sc0 * d0 + sc1 * d1;
    imn = m0 * bs16[4 * p + h] + m1 * bs16[4 * p + 2 + h];
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        isc += __shfl_xor(isc, o, 64);
        imn += __shfl_xor(imn, o, 64);
    }
}

X100_DEV float q4k_combine(const v4i &hdr, float dx, int isc, int imn)
{
    const uint32_t h0 = (uint32_t)hdr[0];
    const float d = h2f((uint16_t)(h0 & 0xffff)), dmin = h2f((uint16_t)(h0 >> 16));
    const float dd = dx * d, dm = dx * dmin;
    return dd * (float)isc - dm * (float)imn;
}

X100_DEV float swiglu(float g, float u)
{
    const float e = (float)exp(-(double)g);
    return (g / (1.0f + e)) * u;
}

// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_moe_route(int M, int d, int n_exp, int n_act,
                                                   const float *__restrict__ hn,
                                                   const float *__restrict__ R, MoeWs ws,
                                                   int *__restrict__ sel_out,
                                                   float *__restrict__ sw_out)
{
    __shared__ int s_last;
    __shared__ int s_sel[8 * 8];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nsb = d / 256;

    // Router logits, one wave per expert (qwen_moe.c:296).
    const int e = blockIdx.x * 4 + w;
    if (e < n_exp) {
        const float *rw = R + (size_t)e * d;
        for (int m = 0; m < M; m++) {
            const float *h = hn + (size_t)m * d;
            float s = 0.0f;
            for (int k = 4 * lane; k < d; k += 256) {
                const float4 a = *(const float4 *)(rw + k);
                const float4 b = *(const float4 *)(h + k);
                s += a.x * b.x;
                s += a.y * b.y;
                s += a.z * b.z;
                s += a.w * b.w;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            if (lane == 0) ws.logits[m * n_exp + e] = s;
        }
    }
    // Q8_K of the hn rows (input of every expert's gate/up).
    for (int q = blockIdx.x * 4 + w; q < M * nsb; q += gridDim.x * 4)
        q8k_block_wave(hn + (size_t)q * 256, ws.xq + (size_t)q * 256, ws.xbs + q * 16, ws.xd + q);

    __threadfence();  // every thread releases its own writes before the block is counted
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(ws.cnt_route, 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // Softmax over all experts, top-n_act by repeated argmax (ties -> lower index), renormalise
    // (qwen_moe.c:298-301).  One wave per token row; lane l holds experts l, l+64, l+128, l+192.
    for (int m = w; m < M; m += 4) {
        float p[4];
        float mx = -1e30f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int ex = lane + 64 * c;
            p[c] = ex < n_exp ? ws.logits[m * n_exp + ex] : -1e30f;
            mx = fmaxf(mx, p[c]);
        }
        mx = wave_max_f(mx);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int ex = lane + 64 * c;
            p[c] = ex < n_exp ? (float)exp((double)(p[c] - mx)) : 0.0f;
            s += p[c];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        const float inv = 1.0f / s;
        // Probabilities are >= 0 (NaN from bad input is treated as 0), used/absent experts -2, so
        // every pass below selects a distinct valid expert.
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float pv = p[c] * inv;
            p[c] = (lane + 64 * c) < n_exp ? (pv == pv ? pv : 0.0f) : -2.0f;
        }

        float wsel[8];
        int isel[8];
        for (int a = 0; a < n_act; a++) {
            float bv = -1.0f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int ex = lane + 64 * c;
                if (p[c] > bv) { bv = p[c]; bi = ex; }   // c ascending: lower index kept on ties
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            wsel[a] = bv;
            isel[a] = bi;
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (lane + 64 * c == bi) p[c] = -2.0f;
        }
        if (lane == 0) {
            float ssum = 0.0f;
            for (int a = 0; a < n_act; a++) ssum += wsel[a];
            for (int a = 0; a < n_act; a++) {
                const float wv = wsel[a] / ssum;
                s_sel[m * n_act + a] = isel[a];
                ws.sel[m * n_act + a] = isel[a];
                ws.sw[m * n_act + a] = wv;
                if (sel_out) sel_out[m * n_act + a] = isel[a];
                if (sw_out) sw_out[m * n_act + a] = wv;
            }
        }
    }
    __syncthreads();
    // Expert union: union slot per distinct expert, with the (row, slot) pairs that use it.
    if (threadIdx.x == 0) {
        int U = 0;
        for (int pr = 0; pr < M * n_act; pr++) {
            const int ex = s_sel[pr];
            int u = 0;
            while (u < U && ws.uniq[u] != ex) u++;
            if (u == U) {
                ws.uniq[U] = ex;
                ws.ucnt[U] = 0;
                U++;
            }
            if (ws.ucnt[u] < 8) {   // distinct experts per row => at most M <= 8 pairs
                ws.upairs[u * 8 + ws.ucnt[u]] = pr;
                ws.ucnt[u]++;
            }
        }
        *ws.nuniq = U;
        *ws.cnt_route = 0;
    }
}

// ------------------------------------------------------------------------------------------------
// grid (U_max, ff / GU_ROWS).  Units (matrix g/u, row, super-block) = 2*GU_ROWS*nsb, 8 lanes each.
template <int UPL>
__global__ __launch_bounds__(256) void k_moe_gate_up(int M, int d, int ff, int n_act,
                                                     const uint8_t *__restrict__ Wg,
                                                     const uint8_t *__restrict__ Wu, MoeWs ws)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int s_pairs[8], s_cnt, s_last;
    const int u = blockIdx.x;
    if (u >= *ws.nuniq) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 7;
    const int nsb = d / 256;
    const int ex = ws.uniq[u], cnt = ws.ucnt[u];
    const int r0 = blockIdx.y * GU_ROWS;
    const int nunits = 2 * GU_ROWS * nsb;
    const size_t erow = (size_t)nsb * 144;               // bytes per row
    const size_t emat = erow * ff;                        // bytes per expert matrix

    v4i hdr[UPL], qs[UPL];
#pragma unroll
    for (int c = 0; c < UPL; c++) {
        const int un = c * 32 + w * 8 + (lane >> 3);
        if (un < nunits) {
            const int mat = un / (GU_ROWS * nsb), rem = un - mat * GU_ROWS * nsb;
            const int r = rem / nsb, sb = rem - r * nsb;
            const uint8_t *blk = (mat ? Wu : Wg) + ex * emat + (size_t)(r0 + r) * erow + sb * 144;
            hdr[c] = *(const v4i *)blk;
            qs[c] = *(const v4i *)(blk + 16 + 16 * i);
        } else {
            hdr[c] = qs[c] = v4i{0, 0, 0, 0};
        }
    }

    // Q8_K of the hn rows of this expert's pairs -> LDS.
    int8_t *xq = (int8_t *)smem;                    // [8][nsb][256]
    int *xbs = (int *)(xq + 8 * nsb * 256);         // [8][nsb][16]
    float *xd = (float *)(xbs + 8 * nsb * 16);      // [8][nsb]
    float *tv = xd + 8 * nsb;                       // [8][2][GU_ROWS][nsb]
    if (threadIdx.x < 8) s_pairs[threadIdx.x] = threadIdx.x < cnt ? ws.upairs[u * 8 + threadIdx.x] : 0;
    if (threadIdx.x == 0) s_cnt = cnt;
    __syncthreads();
    for (int t = threadIdx.x; t < cnt * nsb * 64; t += 256) {
        const int k = t / (nsb * 64), rem = t - k * nsb * 64;
        const int m = s_pairs[k] / n_act;
        ((uint32_t *)xq)[k * nsb * 64 + rem] = ((const uint32_t *)ws.xq)[m * nsb * 64 + rem];
    }
    for (int t = threadIdx.x; t < cnt * nsb * 16; t += 256) {
        const int k = t / (nsb * 16), rem = t - k * nsb * 16;
        xbs[k * nsb * 16 + rem] = ws.xbs[(s_pairs[k] / n_act) * nsb * 16 + rem];
    }
    for (int t = threadIdx.x; t < cnt * nsb; t += 256) {
        const int k = t / nsb, rem = t - k * nsb;
        xd[k * nsb + rem] = ws.xd[(s_pairs[k] / n_act) * nsb + rem];
    }
    __syncthreads();

#pragma unroll
    for (int c = 0; c < UPL; c++) {
        const int un = c * 32 + w * 8 + (lane >> 3);
        const bool valid = un < nunits;
        const int sb = valid ? un % nsb : 0;
        for (int k = 0; k < cnt; k++) {
            int isc, imn;
            q4k_unit_dot(hdr[c], qs[c], xq + (k * nsb + sb) * 256, xbs + (k * nsb + sb) * 16, i, isc, imn);
            if (valid && i == 0) tv[k * 2 * GU_ROWS * nsb + un] = q4k_combine(hdr[c], xd[k * nsb + sb], isc, imn);
        }
    }
    __syncthreads();

    // g, u sequential over super-blocks; SwiGLU (qwen_moe.c:309).
    for (int t = threadIdx.x; t < cnt * GU_ROWS; t += 256) {
        const int k = t / GU_ROWS, r = t - k * GU_ROWS;
        const float *tg = tv + k * 2 * GU_ROWS * nsb + r * nsb;
        const float *tu = tg + GU_ROWS * nsb;
        float g = 0.0f, up = 0.0f;
        for (int sb = 0; sb < nsb; sb++) g = g + tg[sb];
        for (int sb = 0; sb < nsb; sb++) up = up + tu[sb];
        ws.act[(size_t)s_pairs[k] * ff + r0 + r] = swiglu(g, up);
    }

    // The last block of this expert quantizes the expert's activations to Q8_K.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(&ws.cnt_gu[u], 1) == (int)gridDim.y - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int nsf = ff / 256;
    for (int q = w; q < s_cnt * nsf; q += 4) {
        const int k = q / nsf, sb = q - k * nsf;
        const int pr = s_pairs[k];
        q8k_block_wave(ws.act + (size_t)pr * ff + sb * 256, ws.aq + ((size_t)pr * nsf + sb) * 256,
                       ws.abs_ + (pr * nsf + sb) * 16, ws.ad + pr * nsf + sb);
    }
    if (threadIdx.x == 0) ws.cnt_gu[u] = 0;
}

// ------------------------------------------------------------------------------------------------
// grid (U_max, d / DN_ROWS).  Units (row, super-block) = DN_ROWS*nsf, 8 lanes each.
template <int UPL>
__global__ __launch_bounds__(256) void k_moe_down(int M, int d, int ff, int n_act,
                                                  const uint8_t *__restrict__ Wd, MoeWs ws,
                                                  float *__restrict__ out, int residual)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int s_pairs[8], s_last;
    const int u = blockIdx.x;
    const int U = *ws.nuniq;
    if (u >= U) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 7;
    const int nsf = ff / 256;
    const int ex = ws.uniq[u], cnt = ws.ucnt[u];
    const int r0 = blockIdx.y * DN_ROWS;
    const int nunits = DN_ROWS * nsf;
    const size_t erow = (size_t)nsf * 144;
    const size_t emat = erow * d;

    v4i hdr[UPL], qs[UPL];
#pragma unroll
    for (int c = 0; c < UPL; c++) {
        const int un = c * 32 + w * 8 + (lane >> 3);
        if (un < nunits) {
            const int r = un / nsf, sb = un - r * nsf;
            const uint8_t *blk = Wd + ex * emat + (size_t)(r0 + r) * erow + sb * 144;
            hdr[c] = *(const v4i *)blk;
            qs[c] = *(const v4i *)(blk + 16 + 16 * i);
        } else {
            hdr[c] = qs[c] = v4i{0, 0, 0, 0};
        }
    }

    int8_t *aq = (int8_t *)smem;                    // [8][nsf][256]
    int *abs_ = (int *)(aq + 8 * nsf * 256);        // [8][nsf][16]
    float *ad = (float *)(abs_ + 8 * nsf * 16);     // [8][nsf]
    float *tv = ad + 8 * nsf;                       // [8][DN_ROWS][nsf]
    if (threadIdx.x < 8) s_pairs[threadIdx.x] = threadIdx.x < cnt ? ws.upairs[u * 8 + threadIdx.x] : 0;
    __syncthreads();
    for (int t = threadIdx.x; t < cnt * nsf * 64; t += 256) {
        const int k = t / (nsf * 64), rem = t - k * nsf * 64;
        ((uint32_t *)aq)[k * nsf * 64 + rem] = ((const uint32_t *)ws.aq)[s_pairs[k] * nsf * 64 + rem];
    }
    for (int t = threadIdx.x; t < cnt * nsf * 16; t += 256) {
        const int k = t / (nsf * 16), rem = t - k * nsf * 16;
        abs_[k * nsf * 16 + rem] = ws.abs_[s_pairs[k] * nsf * 16 + rem];
    }
    for (int t = threadIdx.x; t < cnt * nsf; t += 256) {
        const int k = t / nsf, rem = t - k * nsf;
        ad[k * nsf + rem] = ws.ad[s_pairs[k] * nsf + rem];
    }
    __syncthreads();

#pragma unroll
    for (int c = 0; c < UPL; c++) {
        const int un = c * 32 + w * 8 + (lane >> 3);
        const bool valid = un < nunits;
        const int sb = valid ? un % nsf : 0;
        for (int k = 0; k < cnt; k++) {
            int isc, imn;
            q4k_unit_dot(hdr[c], qs[c], aq + (k * nsf + sb) * 256, abs_ + (k * nsf + sb) * 16, i, isc, imn);
            if (valid && i == 0) tv[k * nunits + un] = q4k_combine(hdr[c], ad[k * nsf + sb], isc, imn);
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < cnt * DN_ROWS; t += 256) {
        const int k = t / DN_ROWS, r = t - k * DN_ROWS;
        float y = 0.0f;
        for (int sb = 0; sb < nsf; sb++) y = y + tv[k * nunits + r * nsf + sb];
        ws.ydn[(size_t)s_pairs[k] * d + r0 + r] = y;
    }

    // The last expert block of this row range combines the slots in order (qwen_moe.c:310-311).
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(&ws.cnt_dn[blockIdx.y], 1) == U - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int t = threadIdx.x; t < M * DN_ROWS; t += 256) {
        const int m = t / DN_ROWS, r = t - m * DN_ROWS;
        const int row = r0 + r;
        float eo = 0.0f;
        for (int a = 0; a < n_act; a++)
            eo = eo + ws.sw[m * n_act + a] * ws.ydn[(size_t)(m * n_act + a) * d + row];
        float *o = out + (size_t)m * d + row;
        *o = residual ? *o + eo : eo;
    }
    if (threadIdx.x == 0) ws.cnt_dn[blockIdx.y] = 0;
}

MoeWs carve(uintptr_t base, int M, int d, int ff, int n_exp, int n_act, size_t *total)
{
    const int P = M * n_act;
    const int nsb = d / 256, nsf = ff / 256;
    size_t off = 0;
    MoeWs ws;
    auto take = [&](size_t bytes) {
        void *r = (void *)(base + off);
        off += al(bytes);
        return r;
    };
    // Counters first so that a zero-filled fresh workspace has them at 0.
    ws.cnt_route = (int *)take(sizeof(int));
    ws.cnt_gu = (int *)take(sizeof(int) * 64);
    ws.cnt_dn = (int *)take(sizeof(int) * 4096);
    ws.logits = (float *)take(sizeof(float) * M * n_exp);
    ws.sel = (int *)take(sizeof(int) * P);
    ws.sw = (float *)take(sizeof(float) * P);
    ws.nuniq = (int *)take(sizeof(int));
    ws.uniq = (int *)take(sizeof(int) * P);
    ws.ucnt = (int *)take(sizeof(int) * P);
    ws.upairs = (int *)take(sizeof(int) * P * 8);
    ws.xq = (int8_t *)take((size_t)M * nsb * 256);
    ws.xbs = (int *)take(sizeof(int) * M * nsb * 16);
    ws.xd = (float *)take(sizeof(float) * M * nsb);
    ws.act = (float *)take(sizeof(float) * (size_t)P * ff);
    ws.aq = (int8_t *)take((size_t)P * nsf * 256);
    ws.abs_ = (int *)take(sizeof(int) * P * nsf * 16);
    ws.ad = (float *)take(sizeof(float) * P * nsf);
    ws.ydn = (float *)take(sizeof(float) * (size_t)P * d);
    if (total) *total = off;
    return ws;
}

}  // namespace

size_t x100_moe_workspace_bytes(int M, int d, int ff, int n_exp, int n_act)
{
    size_t total = 0;
    carve(0, M, d, ff, n_exp, n_act, &total);
    return total;
}

hipError_t x100_moe_launch(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                           const void *Wg, const void *Wu, const void *Wd, float *out, int residual,
                           int *sel, float *sw, void *workspace, hipStream_t s)
{
    if (M < 1 || M > 8 || n_act < 1 || n_act > 8 || n_exp < n_act || n_exp > 256) return hipErrorInvalidValue;
    if (d % 256 || ff % 256 || d / DN_ROWS > 4096 || d % DN_ROWS || ff % GU_ROWS) return hipErrorInvalidValue;
    const int nsb = d / 256, nsf = ff / 256;
    if (2 * GU_ROWS * nsb > 8 * 32 || DN_ROWS * nsf > 8 * 32) return hipErrorInvalidValue;
    MoeWs ws = carve((uintptr_t)workspace, M, d, ff, n_exp, n_act, nullptr);
    const int Umax = min(M * n_act, n_exp);

    hipLaunchKernelGGL(k_moe_route, dim3((n_exp + 3) / 4), dim3(256), 0, s, M, d, n_exp, n_act, hn, R,
                       ws, sel, sw);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;

    const size_t lds_gu = (size_t)8 * nsb * (256 + 64 + 4) + (size_t)8 * 2 * GU_ROWS * nsb * 4;
    const int upl_gu = (2 * GU_ROWS * nsb + 31) / 32;
    const dim3 g_gu(Umax, ff / GU_ROWS);
    const uint8_t *wg = (const uint8_t *)Wg, *wu = (const uint8_t *)Wu;
    switch (upl_gu) {
    case 1: hipLaunchKernelGGL(k_moe_gate_up<1>, g_gu, dim3(256), lds_gu, s, M, d, ff, n_act, wg, wu, ws); break;
    case 2: hipLaunchKernelGGL(k_moe_gate_up<2>, g_gu, dim3(256), lds_gu, s, M, d, ff, n_act, wg, wu, ws); break;
    case 3: case 4: hipLaunchKernelGGL(k_moe_gate_up<4>, g_gu, dim3(256), lds_gu, s, M, d, ff, n_act, wg, wu, ws); break;
    default: hipLaunchKernelGGL(k_moe_gate_up<8>, g_gu, dim3(256), lds_gu, s, M, d, ff, n_act, wg, wu, ws); break;
    }
    err = hipGetLastError();
    if (err != hipSuccess) return err;

    const size_t lds_dn = (size_t)8 * nsf * (256 + 64 + 4) + (size_t)8 * DN_ROWS * nsf * 4;
    const int upl_dn = (DN_ROWS * nsf + 31) / 32;
    const dim3 g_dn(Umax, d / DN_ROWS);
    const uint8_t *wd = (const uint8_t *)Wd;
    switch (upl_dn) {
    case 1: hipLaunchKernelGGL(k_moe_down<1>, g_dn, dim3(256), lds_dn, s, M, d, ff, n_act, wd, ws, out, residual); break;
    case 2: hipLaunchKernelGGL(k_moe_down<2>, g_dn, dim3(256), lds_dn, s, M, d, ff, n_act, wd, ws, out, residual); break;
    case 3: case 4: hipLaunchKernelGGL(k_moe_down<4>, g_dn, dim3(256), lds_dn, s, M, d, ff, n_act, wd, ws, out, residual); break;
    default: hipLaunchKernelGGL(k_moe_down<8>, g_dn, dim3(256), lds_dn, s, M, d, ff, n_act, wd, ws, out, residual); break;
    }
    return hipGetLastError();
}
