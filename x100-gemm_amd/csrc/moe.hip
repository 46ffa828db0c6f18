// Qwen3-MoE decode layer (the FFN block of qwen_moe.c:294-311) for M token rows: the kernels below
// for up to 8 rows, and from 9 rows (moe_launch_mfma) the (row, slot) pairs grouped by expert into
// chunks of 32 on the matrix cores (k_moe_mfma).  Both give each row the same bits as a one-row
// call.
//
// Up to 8 rows, three or four launches on one stream; each kernel only reads what an earlier launch
// wrote, so no block ever waits for, or signals, another block (no fences, no atomics):
//   k_moe_route       router logits R.hn (one wave per expert and token row) and the Q8_K form of
//                     every hn row.  In a decoder layer at d = 2048, k_moe_route_norm instead: the row
//                     hn = rmsnorm(h + o) formed in every block first, and the residual add of o
//                     left to the combine.
//   k_moe_gate_up_p   persistent blocks over the work items (union slot, GU_ROWS rows of ff).  Every
//                     block derives the routing of all rows itself (cheaper than another launch;
//                     block 0 publishes it), then streams the items' rows of the expert's gate and
//                     up matrices once for all token rows that chose the expert (Q4_K x Q8_K, the
//                     MUL_MAT_ID grouping of ime.cpp:667-697), the next item's weights in flight
//                     while the current one is computed, and writes SwiGLU(g, u) per (token row,
//                     slot) pair.
//   k_moe_down_fused  grid (FD_DN rows of d, row groups of at most 32 pairs): every pair's
//                     activation row quantized to Q8_K in LDS, the down projection of those rows
//                     for the group's pairs, and the weighted combine in slot order, written to out.
//   k_moe_down        (when the fused form does not fit: large ff) grid (union slot, DN_ROWS rows
//   + k_moe_combine   of d): the expert's activation rows in Q8_K, down projection, y per pair;
//                     then out[m] (+)= sum_a w_a * y_a.
#include "x100_common.h"
#include "x100_internal.h"

namespace {

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr int GU_ROWS = 8;    // gate/up rows of ff per work item
constexpr int GU_NWV = 4;     // waves per block of k_moe_gate_up_p (one per token row for the routing)
constexpr int DN_ROWS = 16;   // down rows of d per block
constexpr int MF_MIN_ROWS = 9;   // token rows from which the expert products run on the matrix cores

// Workspace layout (device memory owned by the library, sized by x100_moe_workspace_bytes).
struct MoeWs {
    float *logits;        // [M][n_exp]
    int *sel;             // [M][n_act]
    float *sw;            // [M][n_act]
    int *nuniq;           // [1]
    int *uniq;            // [P]          expert id of union slot u (P = M*n_act)
    int *ucnt;            // [P]          pairs in union slot u
    int *upairs;          // [slot][8] pair ids (m*n_act + a) of union slot u, m ascending (up to
                          // 8 rows); [chunk][32] from 9 rows (chunks of up to 32 pairs per expert)
    uint8_t *xrec;        // Q8_K of the hn rows: up to 8 rows the records [M][nsb] (KREC bytes
                          // each, x100_common.h); from 9 rows [M][rec] = q[nsb][256] |
                          // bsum[nsb][16] (int) | d[nsb] (float), rec rounded up to 16 bytes
    float *act;           // [P][ff]
    float *ydn;           // [P][d]
    uint8_t *xact;        // [P][recf]: Q8_K of act row p (9 or more token rows), layout of xrec
};

inline size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

// Expert weight layouts.  GGUF (TL = false): row-major, 144-byte Q4_K blocks, row r's super-block
// sb at (r * nsb + sb) * 144.  Tiled (TL = true, written by k_moe_tile_pack): the same bytes
// regrouped in tiles of 8 rows x one super-block (1152 bytes), tiles row-group major; inside a
// tile, 16-byte granule g (0: the header d, dmin, scales; 1..8: qs bytes 16(g-1) .. +16) of row
// r & 7 at 128 g + 16 (r & 7).  The 8 rows of a granule fill one 128-byte cache line, so a wave
// reading granule g of 32 rows touches 4 whole lines instead of 32 partial ones, and the 8 rows
// of a row group stay one contiguous span (nsb tiles), as in the GGUF layout.
// Byte offset of granule g of row r, super-block sb, in a matrix of nsb super-blocks per row.
template <bool TL>
X100_DEV size_t q4k_gofs(size_t r, int sb, int g, int nsb)
{
    if constexpr (TL)
        return (((r >> 3) * nsb + sb) * 9 + g) * 128 + 16 * (r & 7);
    else
        return (r * nsb + sb) * 144 + 16 * g;
}
// A unit's header and lane half h's qs granules (4h + 1 .. 4h + 4, in qv[0..3]) from weights
// staged in LDS in the layout of TL: blk = the unit's 144-byte block (GGUF), or its granule 0
// (tiled; the callers give the 8 units of 16 consecutive lanes the 8 rows of one tile, so that
// each read of the 16 lanes covers 128 contiguous bytes per lane half).  Reading lane half 1's
// granules rotated by one (so that the halves fall in opposite 128-byte halves of a 256-byte LDS
// line) and restoring the order with selects measured slower: M = 1 19.4 us against 15.6 us.
template <bool TL>
X100_DEV void q4k_lds_unit(const uint8_t *blk, int h, v4i &hdr, v4i (&qv)[4])
{
    hdr = *(const v4i *)blk;
    if constexpr (TL) {
#pragma unroll
        for (int pc = 0; pc < 4; pc++) qv[pc] = *(const v4i *)(blk + 128 * (1 + 4 * h + pc));
    } else {
#pragma unroll
        for (int pc = 0; pc < 4; pc++) qv[pc] = *(const v4i *)(blk + 16 + 64 * h + 16 * pc);
    }
}

// Bytes of one row's Q8_K record (nsb 256-element blocks).
__host__ __device__ inline int q8k_rec_bytes(int nsb) { return (nsb * (256 + 64 + 4) + 15) & ~15; }

// get_scale_min_k4 (repack.cpp:222-233) over the header dwords 1..3 of a Q4_K block.
X100_DEV uint32_t hbyte(const v4i &h, int k)
{
    const uint32_t w = (uint32_t)(k < 4 ? h[1] : (k < 8 ? h[2] : h[3]));
    return (w >> (8 * (k & 3))) & 0xffu;
}
X100_DEV void gsm(const v4i &h, int j, int &sc, int &m)
{
    // Both forms computed and selected (j is lane-dependent: no branch in the unrolled loops);
    // byte indices modulo 12 keep every read inside the 12 scale bytes.
    const uint32_t bj = hbyte(h, j), bj4 = hbyte(h, (j + 4) % 12), bjm4 = hbyte(h, (j + 8) % 12);
    sc = j < 4 ? (int)(bj & 63) : (int)((bj4 & 0xf) | ((bjm4 >> 6) << 4));
    m = j < 4 ? (int)(bj4 & 63) : (int)((bj4 >> 4) | ((bj >> 6) << 4));
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
    isc = sum8_i(sc0 * d0 + sc1 * d1);
    imn = sum8_i(m0 * bs16[4 * p + h] + m1 * bs16[4 * p + 2 + h]);
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
// Router.  Wave g < n_exp * M computes the logit of expert g / M for token row g % M (qwen_moe.c:296;
// lane l sums elements 4l..4l+3, +256, ... in order, then a butterfly over the lanes), one row per
// wave so that no wave runs the dependent add chains of several rows; the following waves quantize
// four 256-element blocks of hn each into the Q8_K records ws.xrec[m * nsb + sb].  Blocks of
// RT_WPB = 2 waves, so that the 128 router waves of one token row spread over 64 CUs (each CU
// pulls its router rows and hn through its own load path): M = 1 15.85 -> 15.67 us against 4
// waves per block; 1 wave per block was as fast at M = 1 but slower at M = 4.  A block that holds
// both kinds of wave (n_exp * M odd) works as before: its quantizer wave loads no router row, takes
// part in the hn DMA and the barrier, and skips the dot.  A block stages only the hn rows of its
// own waves (at most RT_WPB rows; all M rows had made M = 8 1.5 us slower: 64 KiB of DMA per block).
// ------------------------------------------------------------------------------------------------
constexpr int RT_WPB = 2;
__global__ __launch_bounds__(64 * RT_WPB) void k_moe_route(int M, int d, int n_exp, uint32_t mnsb, const float *__restrict__ hn,
                                                   const float *__restrict__ R, MoeWs ws)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float4 *s_hn = (float4 *)smem;   // [min(M, RT_WPB)][d/4]: the hn rows of the block's router waves
    const int lane = threadIdx.x & 63;
    const int g0 = blockIdx.x * RT_WPB, wave = g0 + wave_id();
    const int nsb = d / 256, nq = M * nsb, nrw = n_exp * M;
    // wave g works on token row g % M, so the block's waves need rows g0 % M, (g0 + 1) % M, ...:
    // min(M, RT_WPB) of them

    if (wave >= nrw) {   // quantizer waves (wave-uniform)
        const int qb = 4 * (wave - nrw);
        if (qb < nq) {
            float4 v[4];
            q8k_load(buf_rsrc(hn, (uint32_t)(M * d) * 4u), d, nsb, mnsb, nq, qb, v);
            q8k_quant(v, nq, qb, ws.xrec);
        }
        if (RT_WPB * (int)blockIdx.x >= nrw) return;   // a block of quantizer waves only
    }

    // The wave's expert and token row, and its router row (elements past d read as 0 and are not
    // used; none for quantizer waves).
    const int gw = min(wave, nrw - 1), e = gw / M, m = gw - e * M;
    const rsrc_t rr = buf_rsrc(R + (size_t)e * d, wave < nrw ? (uint32_t)d * 4u : 0u);
    float4 rv[16];
#pragma unroll
    for (int j = 0; j < 16; j++) rv[j] = buf_load_f4(rr, (uint32_t)(4 * lane + 256 * j) * 4u);

    // hn -> LDS (the block's rows: nrb * d/256 chunks of 1 KiB, one wave each), asynchronous.  Up to
    // RT_WPB rows these are all M rows in order (slot = row); above, slot i holds row (g0 + i) % M.
    if (M <= RT_WPB) {
        for (int ch = wave_id(); ch < M * nsb; ch += RT_WPB)
            dma_1k(hn + (size_t)ch * 256 + 4 * lane, smem + ch * 1024);
    } else {
        const int r0 = g0 % M;
        for (int ch = wave_id(); ch < RT_WPB * nsb; ch += RT_WPB) {
            const int sl = (int)udiv16((uint32_t)ch, (uint32_t)nsb, mnsb), r = r0 + sl;
            dma_1k(hn + (size_t)(r < M ? r : r - M) * d + (ch - sl * nsb) * 256 + 4 * lane, smem + ch * 1024);
        }
    }
    __syncthreads();

    if (wave < nrw) {
        const float4 *h = s_hn + (M <= RT_WPB ? m : wave_id()) * (d / 4);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < nsb) {
                const float4 hv = h[lane + 64 * j];
                sum += rv[j].x * hv.x;
                sum += rv[j].y * hv.y;
                sum += rv[j].z * hv.z;
                sum += rv[j].w * hv.w;
            }
        sum = wave_sum_bfly_f(sum);
        if (lane == 0) ws.logits[m * n_exp + e] = sum;
    }
}

// ------------------------------------------------------------------------------------------------
// A decoder layer's step before the MoE block, folded into the router (one token row, d = 2048):
// every 128-thread block forms hn = rmsnorm(h + o, nrm) itself with the operations and order of
// k_rmsnorm<1024> (attn.hip): virtual thread T < 1024 sums (h + o)[T]^2 and (h + o)[T + 1024]^2
// from 0, the 64 virtual threads of a virtual wave reduce by wave_sum_bfly_f's butterfly, the 16
// wave sums are added in order, s = 1 / sqrtf(sum / 2048 + eps) and hn = (h + o) * s * nrm.
// Thread t holds virtual threads 8t .. 8t+7, so virtual lane 8 (t % 8) + j meets its partners
// l^32, l^16, l^8 in threads t^4, t^2, t^1 and l^4, l^2, l^1 inside the thread.
// ------------------------------------------------------------------------------------------------
X100_DEV void rms_row_2048_128(const float *__restrict__ h, const float *__restrict__ o,
                               const float *__restrict__ nrm, float eps, float *s_hn, float *red)
{
    const int t = threadIdx.x;
    float a[8], b[8];
    float4 g[4];   // the norm weights of the thread's elements, loaded with h and o
#pragma unroll
    for (int k = 0; k < 2; k++) {
        g[k] = *(const float4 *)(nrm + 8 * t + 4 * k);
        g[2 + k] = *(const float4 *)(nrm + 1024 + 8 * t + 4 * k);
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const float4 ha = *(const float4 *)(h + 8 * t + 4 * k), oa = *(const float4 *)(o + 8 * t + 4 * k);
        const float4 hb = *(const float4 *)(h + 1024 + 8 * t + 4 * k);
        const float4 ob = *(const float4 *)(o + 1024 + 8 * t + 4 * k);
        a[4 * k] = ha.x + oa.x; a[4 * k + 1] = ha.y + oa.y; a[4 * k + 2] = ha.z + oa.z; a[4 * k + 3] = ha.w + oa.w;
        b[4 * k] = hb.x + ob.x; b[4 * k + 1] = hb.y + ob.y; b[4 * k + 2] = hb.z + ob.z; b[4 * k + 3] = hb.w + ob.w;
    }
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        v[j] = 0.0f + a[j] * a[j];
        v[j] += b[j] * b[j];
    }
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] += __shfl_xor(v[j], 4, 64);   // virtual l^32: thread t^4
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] += dpp_f<0x4E>(0.0f, v[j]);   // virtual l^16: t^2
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] += dpp_f<0xB1>(0.0f, v[j]);   // virtual l^8: t^1
    const float w0 = v[0] + v[4], w1 = v[1] + v[5], w2 = v[2] + v[6], w3 = v[3] + v[7];   // l^4
    const float x0 = w0 + w2, x1 = w1 + w3;                                                 // l^2
    if ((t & 7) == 0) red[t >> 3] = x0 + x1;                                               // l^1
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) tot += red[k];
    const float sc = 1.0f / sqrtf(tot / 2048.0f + eps);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const float4 ga = g[k], gb = g[2 + k];
        *(float4 *)(s_hn + 8 * t + 4 * k) = make_float4(a[4 * k] * sc * ga.x, a[4 * k + 1] * sc * ga.y,
                                                        a[4 * k + 2] * sc * ga.z, a[4 * k + 3] * sc * ga.w);
        *(float4 *)(s_hn + 1024 + 8 * t + 4 * k) = make_float4(b[4 * k] * sc * gb.x, b[4 * k + 1] * sc * gb.y,
                                                               b[4 * k + 2] * sc * gb.z, b[4 * k + 3] * sc * gb.w);
    }
    __syncthreads();
}

// k_moe_route for one token row with the pre-MoE step folded in: hn = rmsnorm(h + o, nrm) in every
// block's LDS (rms_row_2048_128), then wave g < n_exp computes expert g's logit and the waves past
// them quantize the row's Q8_K records, with k_moe_route's operations.  d = 2048, blocks of 2 waves.
__global__ __launch_bounds__(64 * RT_WPB) void k_moe_route_norm(int n_exp, const float *__restrict__ h,
                                                                const float *__restrict__ o,
                                                                const float *__restrict__ nrm, float eps,
                                                                const float *__restrict__ R, MoeWs ws)
{
    static_assert(RT_WPB == 2, "rms_row_2048_128 takes 128 threads");
    __shared__ __attribute__((aligned(16))) float s_hn[2048];
    __shared__ float red[16];
    constexpr int d = 2048, nsb = 8;
    const int lane = threadIdx.x & 63, wave = blockIdx.x * RT_WPB + wave_id();
    // the router row first: these are the kernel's critical loads (none for quantizer waves)
    const int e = min(wave, n_exp - 1);
    const rsrc_t rr = buf_rsrc(R + (size_t)e * d, wave < n_exp ? (uint32_t)d * 4u : 0u);
    float4 rv[nsb];
#pragma unroll
    for (int j = 0; j < nsb; j++) rv[j] = buf_load_f4(rr, (uint32_t)(4 * lane + 256 * j) * 4u);
    rms_row_2048_128(h, o, nrm, eps, s_hn, red);
    if (wave >= n_exp) {   // quantizer waves (wave-uniform): records 4 (wave - n_exp) .. +3
        const int qb = 4 * (wave - n_exp), q = qb + (lane >> 4);
        if (qb < nsb) {
            float4 v[4];
#pragma unroll
            for (int c = 0; c < 4; c++)
                v[c] = q < nsb ? *(const float4 *)(s_hn + q * 256 + 16 * (lane & 15) + 4 * c) : make_float4(0, 0, 0, 0);
            q8k_quant(v, nsb, qb, ws.xrec);
        }
        return;
    }
    const float4 *hv4 = (const float4 *)s_hn;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < nsb; j++) {
        const float4 hv = hv4[lane + 64 * j];
        sum += rv[j].x * hv.x;
        sum += rv[j].y * hv.y;
        sum += rv[j].z * hv.z;
        sum += rv[j].w * hv.w;
    }
    sum = wave_sum_bfly_f(sum);
    if (lane == 0) ws.logits[e] = sum;
}

// ------------------------------------------------------------------------------------------------
// Router of many token rows: the logits of k_moe_route (same per-lane order and butterfly, so the
// same bits) from blocks of RR_ROWS token rows x 4 * epw experts, so that each loaded hn row serves
// up to 32 experts instead of 4 (epw grows with M: more experts per block, fewer blocks).  Wave w
// computes experts 4 * epw * bx + epw * w .. +epw.  Blocks bx >= ceil(n_exp / (4 * epw)) quantize
// the chunk's hn rows to Q8_K (one wave per 256-element block, from global memory).
// grid (ceil(n_exp / (4 * epw)) + ceil(RR_ROWS * d / 1024), ceil(M / RR_ROWS)).
// ------------------------------------------------------------------------------------------------
constexpr int RR_ROWS = 4;

// NJ: 256-element blocks of d held per lane (d <= 256 * NJ); EXACT: d == 256 * NJ, so the block
// loop needs no range tests (a test per block split each dot into branches and kept the RB rows'
// sums from interleaving).
template <int NJ, bool EXACT>
__global__ __launch_bounds__(256) void k_moe_route_rows(int M, int d, int n_exp, int epw, const float *__restrict__ hn,
                                                        const float *__restrict__ R, MoeWs ws)
{
    const int lane = threadIdx.x & 63, w = wave_id();
    const int nsb = EXACT ? NJ : d / 256;
    const int row0 = blockIdx.y * RR_ROWS, nr = min(RR_ROWS, M - row0);
    const int ngrp = (n_exp + 4 * epw - 1) / (4 * epw);
    if ((int)blockIdx.x >= ngrp) {
        const int q = ((int)blockIdx.x - ngrp) * 4 + w;
        if (q >= nr * nsb) return;
        const int m = q / nsb, sb = q - m * nsb;
        const float4 v = *(const float4 *)(hn + (size_t)(row0 + m) * d + sb * 256 + 4 * lane);
        uint8_t *rec = ws.xrec + (size_t)(row0 + m) * q8k_rec_bytes(nsb);
        q8_K_wave(v, (int8_t *)rec + sb * 256, (int *)(rec + nsb * 256) + sb * 16, (float *)(rec + nsb * 320) + sb);
        return;
    }

    // The block's hn rows in registers, RB at a time (all four at d <= 2048), and the wave's router
    // rows streamed through a two-row register ring, the next expert's row loading while the
    // current one's RB dot products run: no LDS, and no load between an expert's dots.
    constexpr int RB = NJ <= 8 ? RR_ROWS : 1;   // hn rows held per pass (RB * NJ float4 registers)
    const int e0 = blockIdx.x * 4 * epw + epw * w;
    auto rload = [&](int e, float4 *rv) {
        const rsrc_t rr = buf_rsrc(R + (size_t)min(e, n_exp - 1) * d, (uint32_t)d * 4u);   // clamped expert
#pragma unroll
        for (int j = 0; j < NJ; j++) rv[j] = buf_load_f4(rr, (uint32_t)(4 * lane + 256 * j) * 4u);
    };
    for (int mb = 0; mb < nr; mb += RB) {
        float4 rv[2][NJ];   // ring: router rows of experts i, i + 1
        rload(e0, rv[0]);
        float4 hv[RB][NJ];
#pragma unroll
        for (int m = 0; m < RB; m++) {
            const rsrc_t hr = buf_rsrc(hn + (size_t)(row0 + min(mb + m, nr - 1)) * d, (uint32_t)d * 4u);
#pragma unroll
            for (int j = 0; j < NJ; j++) hv[m][j] = buf_load_f4(hr, (uint32_t)(4 * lane + 256 * j) * 4u);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = e0 + i;
            if (i >= epw) break;
            if (i + 1 < epw) rload(e + 1, rv[(i + 1) & 1]);
            if (e < n_exp) {
                // each row's sum in k_moe_route's order (blocks j ascending, then x, y, z, w); the
                // RB rows' independent sums interleaved
                float sum[RB];
#pragma unroll
                for (int m = 0; m < RB; m++) sum[m] = 0.0f;
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    if (EXACT || j < nsb) {
#pragma unroll
                        for (int m = 0; m < RB; m++) sum[m] += rv[i & 1][j].x * hv[m][j].x;
#pragma unroll
                        for (int m = 0; m < RB; m++) sum[m] += rv[i & 1][j].y * hv[m][j].y;
#pragma unroll
                        for (int m = 0; m < RB; m++) sum[m] += rv[i & 1][j].z * hv[m][j].z;
#pragma unroll
                        for (int m = 0; m < RB; m++) sum[m] += rv[i & 1][j].w * hv[m][j].w;
                    }
#pragma unroll
                for (int m = 0; m < RB; m++)
                    if (mb + m < nr) {
                        const float v = wave_sum_bfly_f(sum[m]);
                        if (lane == 0) ws.logits[(size_t)(row0 + mb + m) * n_exp + e] = v;
                    }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Routing of all M rows from the logits, computed identically by every gate/up block.
// Softmax over all experts (max-subtract, exp, times 1/sum; lane l of a wave holds experts
// l, l+64, l+128, l+192 and the sum is lane-partial then butterfly), top-n_act by repeated
// argmax with the lower expert id kept on ties (qwen_moe.c:298-300), renormalise (:301).
// Outputs in LDS: s_sel/s_w [M][n_act] (slot order), s_uniq[U] = distinct experts ascending.
// ------------------------------------------------------------------------------------------------
struct RouteLds {
    __attribute__((aligned(16))) int sel[8 * 8];
    float w[8 * 8];
    int uniq[64];
    uint64_t mask[8][4];   // experts chosen by row m: bit l of mask[m][c] = expert 64c + l
    uint64_t umask[4];     // their union
    int U;
};

// Softmax, top-k and expert union of the M token rows (qwen_moe.c:296-301), one wave per row;
// KC = 64-expert groups per lane (2 for n_exp <= 128, else 4).
template <int NWV, int KC, int NE = 0, int NA = 0>
X100_DEV void route_rows(int M, int n_exp_rt, int n_act_rt, const float *__restrict__ logits, RouteLds &rl)
{
    // NE, NA: the expert count and top-k known at compile time (0: taken from the arguments), so
    // that the selection rounds unroll without range tests
    const int n_exp = NE ? NE : n_exp_rt, n_act = NA ? NA : n_act_rt;
    const int lane = threadIdx.x & 63, w = wave_id();
    uint64_t rowmask[KC];   // ballots of the chosen experts of this wave's last row
#pragma unroll
    for (int c = 0; c < KC; c++) rowmask[c] = 0;
    for (int m = w; m < M; m += NWV) {
        bool picked[KC];   // experts lane + 64c chosen for row m
#pragma unroll
        for (int c = 0; c < KC; c++) picked[c] = false;
        float p[KC];
        float mx = -1e30f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int ex = lane + 64 * c;
            const float lv = logits[m * n_exp + min(ex, n_exp - 1)];   // unconditional load
            p[c] = ex < n_exp ? lv : -1e30f;
            mx = fmaxf(mx, p[c]);
        }
        mx = wave_max_u(mx);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int ex = lane + 64 * c;
            p[c] = ex < n_exp ? (float)exp((double)(p[c] - mx)) : 0.0f;
            s += p[c];
        }
        s = wave_sum_bfly_f(s);
        const float inv = 1.0f / s;
        // Selection keys: the bits of the probability (>= 0, so integer order = float order; NaN
        // from bad input is treated as 0); absent or already chosen experts are INT_MIN, so every
        // pass selects a distinct valid expert.
        int key[KC];
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const float pv = p[c] * inv;
            key[c] = (lane + 64 * c) < n_exp ? __float_as_int(pv == pv ? pv : 0.0f) : INT_MIN;
        }
        float wsel[8];
        int isel[8];
#pragma unroll
        for (int a = 0; a < 8; a++) {
            wsel[a] = 0.0f;
            isel[a] = 0;
            if (a < n_act) {
                // Largest probability (wave maximum of the keys), then the lowest expert id holding
                // it: per group c the lowest lane whose key matches (all ones when none does, so
                // the unsigned minimum picks the lowest group that has one).
                int kl = key[0];
#pragma unroll
                for (int c = 1; c < KC; c++) kl = max(kl, key[c]);
                const int km = wave_max_iu(kl);
                unsigned bi = 0xffffffffu;
#pragma unroll
                for (int c = 0; c < KC; c++) {
                    const uint64_t h = __ballot(key[c] == km);
                    bi = min(bi, (unsigned)(__ffsll((unsigned long long)h) - 1) | (unsigned)(64 * c));
                }
                wsel[a] = __int_as_float(km);
                isel[a] = (int)bi;
#pragma unroll
                for (int c = 0; c < KC; c++) {
                    const bool hit = (unsigned)(lane + 64 * c) == bi;
                    picked[c] = picked[c] || hit;
                    key[c] = hit ? INT_MIN : key[c];
                }
            }
        }
        // Renormalise (qwen_moe.c:301): the sum in slot order, then one division per slot, lane a
        // doing slot a.
        float ssum = 0.0f;
#pragma unroll
        for (int a = 0; a < 8; a++)
            if (a < n_act) ssum += wsel[a];
        float mine = wsel[0];
        int mine_e = isel[0];
#pragma unroll
        for (int a = 1; a < 8; a++) {
            mine = lane == a ? wsel[a] : mine;
            mine_e = lane == a ? isel[a] : mine_e;
        }
        if (lane < n_act) {
            rl.w[m * n_act + lane] = mine / ssum;
            rl.sel[m * n_act + lane] = mine_e;
        }
#pragma unroll
        for (int c = 0; c < KC; c++) {
            rowmask[c] = __ballot(picked[c]);
            if (lane == 0) rl.mask[m][c] = rowmask[c];
        }
    }
    // Union slots in ascending expert id: slot of expert e = number of chosen experts below e;
    // the union is the OR of the rows' masks, slots are prefix counts of its bits.
    if (M == 1) {
        // one row: wave 0 holds its masks in registers
        if (w == 0) {
            const uint64_t below = (1ull << lane) - 1ull;
            int base = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint64_t um = c < KC ? rowmask[c < KC ? c : 0] : 0;
                if ((um >> lane) & 1ull) rl.uniq[base + __popcll(um & below)] = lane + 64 * c;
                base += __popcll(um);
                if (lane == 0) rl.umask[c] = um;
            }
            if (lane == 0) rl.U = base;
        }
        __syncthreads();
        return;
    }
    __syncthreads();
    if (w == 0) {
        const uint64_t below = (1ull << lane) - 1ull;
        int base = 0;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            uint64_t um = 0;
            for (int m = 0; m < M; m++) um |= rl.mask[m][c];
            if ((um >> lane) & 1ull) rl.uniq[base + __popcll(um & below)] = lane + 64 * c;
            base += __popcll(um);
            if (lane == 0) rl.umask[c] = um;
        }
#pragma unroll
        for (int c = KC; c < 4; c++)
            if (lane == 0) rl.umask[c] = 0;
        if (lane == 0) rl.U = base;
    }
    __syncthreads();
}
template <int NWV>
X100_DEV void route_block(int M, int n_exp, int n_act, const float *__restrict__ logits, RouteLds &rl)
{
    if (n_exp == 128 && n_act == 8)   // Qwen3-30B-A3B
        route_rows<NWV, 2, 128, 8>(M, n_exp, n_act, logits, rl);
    else if (n_exp <= 128)
        route_rows<NWV, 2>(M, n_exp, n_act, logits, rl);
    else
        route_rows<NWV, 4>(M, n_exp, n_act, logits, rl);
}

// Pair t = (token row m, slot a) of the routing in rl: the union slot of its expert, its place in
// the slot's list (earlier rows that chose the expert come first: token rows ascending) and the
// list length.
X100_DEV void pair_slot(int M, int n_act, const RouteLds &rl, int t, int &slot, int &pos, int &cnt)
{
    const int e = rl.sel[t], m = t / n_act, c = e >> 6;
    const uint64_t bit = 1ull << (e & 63);
    slot = __popcll(rl.umask[c] & (bit - 1ull));
    for (int k = 0; k < c; k++) slot += __popcll(rl.umask[k]);
    pos = 0;
    cnt = 0;
    for (int r = 0; r < M; r++) {
        const int has = (rl.mask[r][c] & bit) != 0;
        pos += r < m ? has : 0;
        cnt += has;
    }
}

// Routing of the rows (computed by route_block into rl) -> workspace: sel, sw (and the caller's
// copies), the union (ascending expert id), its pair lists (token row ascending) and size.
X100_DEV void publish_routing(int M, int n_act, const RouteLds &rl, MoeWs ws, int *__restrict__ sel_out,
                              float *__restrict__ sw_out)
{
    const int t = threadIdx.x;
    const int U = rl.U;
    if (t < M * n_act) {
        const int e = rl.sel[t];
        ws.sel[t] = e;
        ws.sw[t] = rl.w[t];
        if (sel_out) sel_out[t] = e;
        if (sw_out) sw_out[t] = rl.w[t];
        int slot, pos, cnt;
        pair_slot(M, n_act, rl, t, slot, pos, cnt);
        ws.upairs[slot * 8 + pos] = t;
        if (pos == 0) {
            ws.uniq[slot] = e;
            ws.ucnt[slot] = cnt;
        }
    }
    if (t == 0) *ws.nuniq = U;
}

// ------------------------------------------------------------------------------------------------
// 9 or more token rows (verify / prefill).  Routing per 8-row chunk of the grid (the same
// route_block as above), written per row; then the pairs (row, slot) are grouped by expert (the
// MUL_MAT_ID grouping of ime.cpp:667-697, qwen_moe_hp.c:1674-1700) into chunks of at most PCH
// pairs per expert, in the union-slot format (uniq, ucnt, upairs) that k_moe_mfma reads.
// Each pair is computed exactly as with one token row, so the order of pairs inside an expert's
// chunks (set by atomics here) does not change any result.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(512) void k_moe_topk_rows(int M, int n_exp, int n_act, MoeWs ws,
                                                       int *__restrict__ sel_out, float *__restrict__ sw_out)
{
    __shared__ RouteLds rl;
    const int row0 = blockIdx.x * 8, Mloc = min(8, M - row0);
    route_block<8>(Mloc, n_exp, n_act, ws.logits + (size_t)row0 * n_exp, rl);
    const int t = threadIdx.x;
    if (t < Mloc * n_act) {
        const int p = row0 * n_act + t;
        ws.sel[p] = rl.sel[t];
        ws.sw[p] = rl.w[t];
        if (sel_out) sel_out[p] = rl.sel[t];
        if (sw_out) sw_out[p] = rl.w[t];
    }
}

// Groups the P pairs (pair p chose expert sel(p)) by expert into chunks of at most PCH: per-expert
// counts by LDS atomics, the chunk base of each expert (exclusive scan of ceil(count / PCH)), then
// each pair placed by an atomic cursor.  Threads 0 .. 255 of the block take part (n_exp <= 256).
template <int PCH, class Sel>
X100_DEV void group_pairs(int P, int n_exp, Sel sel, MoeWs ws)
{
    __shared__ int s_cnt[256], s_cur[256], s_vbase[257];
    const int t = threadIdx.x;
    const bool on = t < 256;
    if (on) {
        s_cnt[t] = 0;
        s_cur[t] = 0;
    }
    // Thread t's pairs t, t + 256, ... (P <= 4096: at most 16) have their experts loaded at once,
    // before the first count: a load per counting step made each step a round trip to memory.
    constexpr int PPT = X100_MOE_MAX_ROWS * 8 / 256;
    int ex[PPT];
#pragma unroll
    for (int i = 0; i < PPT; i++) ex[i] = (on && t + 256 * i < P) ? sel(t + 256 * i) : -1;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PPT; i++)
        if (ex[i] >= 0) atomicAdd(&s_cnt[ex[i]], 1);
    __syncthreads();
    if (t < 64) {
        // chunk bases: exclusive prefix sum of ceil(count / PCH) over the experts, wave 0 with four
        // experts per lane (n_exp <= 256) and a 6-step wave scan, instead of one thread walking them
        int c[4], sum = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = 4 * t + k;
            c[k] = e < n_exp ? (s_cnt[e] + PCH - 1) / PCH : 0;
            sum += c[k];
        }
        int incl = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off, 64);
            if (t >= off) incl += y;
        }
        int v = incl - sum;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = 4 * t + k;
            if (e < n_exp) s_vbase[e] = v;
            v += c[k];
        }
        if (t == 63) {
            s_vbase[n_exp] = incl;
            *ws.nuniq = incl;
        }
    }
    __syncthreads();
    if (t < n_exp) {
        const int c = s_cnt[t], v0 = s_vbase[t];
        for (int k = 0; k * PCH < c; k++) {
            ws.uniq[v0 + k] = t;
            ws.ucnt[v0 + k] = min(PCH, c - PCH * k);
        }
    }
#pragma unroll
    for (int i = 0; i < PPT; i++)
        if (ex[i] >= 0) {
            const int k = atomicAdd(&s_cur[ex[i]], 1);
            ws.upairs[(s_vbase[ex[i]] + k / PCH) * PCH + (k % PCH)] = t + 256 * i;
        }
}

// One block of 256 threads: the grouping of all P pairs from ws.sel.
template <int PCH>
__global__ __launch_bounds__(256) void k_moe_group(int P, int n_exp, MoeWs ws)
{
    group_pairs<PCH>(P, n_exp, [&](int p) { return ws.sel[p]; }, ws);
}


// ------------------------------------------------------------------------------------------------
// Gate/up for 1 .. 8 token rows, persistent: each block derives the routing of all M rows from the
// logits once (route_block, one wave per row, two per wave above 4 rows; block 0 publishes it for
// the down projection and the caller) and stages the Q8_K records of all M rows in LDS (above 4
// rows that makes 2 blocks per CU instead of 3), then walks the work items it =
// blockIdx.x, + gridDim.x, ... (item = union slot u, GU_ROWS rows of ff).  The next item's weights
// are staged into the second of two LDS buffers while the current item is computed, so a block
// always has one item's weights in flight.  An item's expert rows of one matrix are one contiguous
// span, so its DMA walks two spans (gate, then up).  Work units (matrix, row, super-block), two
// lanes each (half h of the Q4_K block), read the weight block and the record from LDS and store
// one fp32 term per token row that chose the expert; g and u are then summed over super-blocks in
// order and SwiGLU(g, u) written per (token row, slot) pair.
// The weight DMA is issued from inline asm (dma16v) and waited for with an exact s_waitcnt: on
// this GPU global stores count in vmcnt too, and only wave 0 stores act (one instruction per item,
// cnt * GU_ROWS <= 64 values), so at the top of an item wave 0 lets its last store stay
// outstanding.
// ------------------------------------------------------------------------------------------------
template <int UPL, int NWV, bool TL>
__global__ __launch_bounds__(64 * NWV) void k_moe_gate_up_p(int M, int d, int ff, int n_exp, int n_act,
                                                            const uint8_t *__restrict__ Wg,
                                                            const uint8_t *__restrict__ Wu, MoeWs ws,
                                                            int *__restrict__ sel_out, float *__restrict__ sw_out)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ RouteLds rl;
    const int nsb = d / 256, P = M * n_act;
    const int t = threadIdx.x, lane = t & 63, w = wave_id(), h = lane & 1;

    // Routing of all rows: rl.uniq holds the union slots' experts (ascending).
    route_block<NWV>(M, n_exp, n_act, ws.logits, rl);

    const int nrg = ff / GU_ROWS, items = rl.U * nrg;
    const int nunits = 2 * GU_ROWS * nsb;
    const size_t erow = (size_t)nsb * 144, emat = erow * ff;
    const int nch = nunits * 9, span = GU_ROWS * nsb * 9;   // 16-byte chunks: item, one matrix
    const uint32_t wbytes = (uint32_t)((nch + 63) / 64 * 1024);
    uint8_t *wl0 = smem + ((size_t)M * nsb * KREC + 1023) / 1024 * 1024;
    float *tv = (float *)(wl0 + 2 * (size_t)wbytes);   // [M][2][GU_ROWS][nsb] + one spare
    int *s_cnt = (int *)(tv + M * 2 * GU_ROWS * nsb + 1);   // [union slot]: its number of pairs
    int *s_pairs = s_cnt + min(P, n_exp);                    // [union slot][8]: its pairs
    const uint32_t wlds = lds_addr(wl0);

    // Weight blocks of item `it` into buffer b: DMA op i copies chunks 64i .. 64i+63 of the gate
    // span then the up span (chunks past the end clamped onto the last one; the buffer is whole KiB).
    auto issue = [&](int it, int b) __attribute__((always_inline)) {
        const int u = it / nrg, r0 = (it - u * nrg) * GU_ROWS;
        const size_t off = (size_t)rl.uniq[u] * emat + (size_t)r0 * erow;
        for (int i = w; i * 64 < nch; i += NWV) {
            const int c = min(i * 64 + lane, nch - 1), mat = c >= span;
            dma16v((mat ? Wu : Wg) + off + 16 * (size_t)(c - mat * span),
                   __builtin_amdgcn_readfirstlane(wlds + b * wbytes + (uint32_t)i * 1024u));
        }
    };
    // The records of all M rows first, then the first item's weights (both waited for at the top
    // of the first item), then each union slot's pair list and size -> LDS.  Records first: every
    // item needs them, and behind the weight requests they arrived later (M = 1 16.0 -> 15.85 us).
    int it = blockIdx.x, b = 0;
    const int totv = M * nsb * KREC / 16;
    for (int ch = w; ch * 64 < totv; ch += NWV)
        dma16v((const v4i *)ws.xrec + min(ch * 64 + lane, totv - 1),
               __builtin_amdgcn_readfirstlane(lds_addr(smem) + (uint32_t)ch * 1024u));
    if (it < items) issue(it, 0);
    if (blockIdx.x == 0) publish_routing(M, n_act, rl, ws, sel_out, sw_out);
    if (t < P) {
        int slot, pos, cnt;
        pair_slot(M, n_act, rl, t, slot, pos, cnt);
        s_pairs[slot * 8 + pos] = t;
        if (pos == 0) s_cnt[slot] = cnt;
    }
    for (bool first = true; it < items; it += gridDim.x, b ^= 1, first = false) {
        // This item's weights are in (this wave's operations; then every wave's, by the barrier),
        // and every wave is done with the other buffer and tv.
        if (w == 0 && !first)
            asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (it + (int)gridDim.x < items) issue(it + gridDim.x, b ^ 1);

        const int u = it / nrg, r0 = (it - u * nrg) * GU_ROWS, cnt = s_cnt[u];
        const uint8_t *wl = wl0 + (size_t)b * wbytes;
        const int tv_spare = M * 2 * GU_ROWS * nsb;
#pragma unroll
        for (int c = 0; c < UPL; c++) {
            // unit un = (matrix, row, super-block) in that order; tiled, the lanes take the units
            // row-fastest (q = (matrix, super-block, row)), so that 8 consecutive lane pairs read
            // the 8 rows of one LDS tile
            const int q = c * 32 * NWV + w * 32 + (lane >> 1);
            const bool valid = q < nunits;
            int un, sb;
            const uint8_t *blk;
            if constexpr (TL) {
                const int qq = valid ? q : 0, rest = qq >> 3, mat = rest / nsb;
                sb = rest - mat * nsb;
                un = (mat * GU_ROWS + (qq & 7)) * nsb + sb;
                blk = wl + (size_t)mat * GU_ROWS * nsb * 144 + sb * 1152 + 16 * (qq & 7);
            } else {
                un = q;
                sb = valid ? un % nsb : 0;
                blk = wl + (size_t)(valid ? un : 0) * 144;
            }
            v4i hdr, qv[4];
            q4k_lds_unit<TL>(blk, h, hdr, qv);
            Q4kHalf uh;
            q4k_scales_gguf(hdr, h, uh);
            q4k_unpack(qv, uh);
            const uint32_t h0 = (uint32_t)hdr[0];
            const float dw = h2f((uint16_t)(h0 & 0xffff)), dmin = h2f((uint16_t)(h0 >> 16));
            for (int k = 0; k < cnt; k++) {
                const uint8_t *rec = smem + (size_t)((s_pairs[u * 8 + k] / n_act) * nsb + sb) * KREC;
                int isc, imn;
                q4k_half_sums(uh, rec, h, isc, imn);
                tv[valid ? k * 2 * GU_ROWS * nsb + un : tv_spare] = q4k_term(dw, dmin, *(const float *)(rec + KR_D), isc, imn);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // g, u sequential over super-blocks; SwiGLU (qwen_moe.c:309): wave 0 only (cnt * GU_ROWS <= 64)
        if (t < cnt * GU_ROWS) {
            const int k = t / GU_ROWS, r = t - k * GU_ROWS;
            const float *tg = tv + k * 2 * GU_ROWS * nsb + r * nsb;
            const float *tu = tg + GU_ROWS * nsb;
            float g = 0.0f, up = 0.0f;
            for (int sb = 0; sb < nsb; sb++) g = g + tg[sb];
            for (int sb = 0; sb < nsb; sb++) up = up + tu[sb];
            ws.act[(size_t)s_pairs[u * 8 + k] * ff + r0 + r] = swiglu(g, up);
        }
    }
    // A block with no item issued the records' DMA and never waited for it: let it land in this
    // block's LDS before the block ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Q8_K of every pair's activation row, once (9 or more token rows): wave q quantizes block
// q % nsf of pair q / nsf with q8_K_wave, into the pair's record of ws.xact.
__global__ __launch_bounds__(256) void k_moe_act_q8k(int P, int ff, MoeWs ws)
{
    const int nsf = ff / 256, q = blockIdx.x * 4 + wave_id(), lane = threadIdx.x & 63;
    if (q >= P * nsf) return;
    const int p = q / nsf, sb = q - p * nsf;
    const float4 v = *(const float4 *)(ws.act + (size_t)p * ff + sb * 256 + 4 * lane);
    uint8_t *rec = ws.xact + (size_t)p * q8k_rec_bytes(nsf);
    q8_K_wave(v, (int8_t *)rec + sb * 256, (int *)(rec + nsf * 256) + sb * 16, (float *)(rec + nsf * 320) + sb);
}

// ------------------------------------------------------------------------------------------------
// Expert-grouped Q4_K x Q8_K products on the matrix cores (many token rows).  The pairs of one
// expert come in chunks of up to 32 (k_moe_group<32>); a wave computes a 32 x 32 tile (chunk pairs
// x weight rows) with v_mfma_i32_32x32x32_i8 per 32-element sub-block j:
//   A = the pairs' Q8_K bytes of sub-block j (lane l: pair l % 32, elements 16 * (l / 32) .. +16),
//   B = the weight rows' 4-bit values of sub-block j times the low or the high 3 bits of the
//       row's 6-bit scale (lane l: row l % 32, the same elements),
// so the two accumulators hold sum_j sc_lo_j dot_j and sum_j sc_hi_j dot_j exactly; a third
// chain whose B holds m_j in every byte gives the min term sum_j m_j * (sum of the activation
// bytes of sub-block j).  These integers equal those of the one-row kernels, and the fp32 combine
// per super-block (q4k_combine) and the sum over super-blocks run in the same order, so every
// output is bit-identical to theirs.
//
// GU: gate and up (A = the hn records, pair p reads row p / n_act); wave w computes matrix w & 1
// (gate, up) for ff rows r0 + 32 * (w >> 1) .. +32, and SwiGLU pairs them through LDS.
// !GU: down projection (A = the activation records of ws.xact, row p); wave w computes d rows
// r0 + 32 * w .. +32.  grid (chunks, ff / 64 or d / 128).
// ------------------------------------------------------------------------------------------------
constexpr int MF_PCH = 32;   // pairs per chunk of the MFMA path
#ifndef MF_DN_RT
#define MF_DN_RT 2           // row tiles per wave of the down projection (one staging part)
#endif
// Super-blocks in the first staged part of k_moe_mfma's activations: all of them up to 4 (one
// staging round trip; the down projection of ff = 768 has 3), else the first half rounded up to
// even, so that the halves meet between two ring steps.
__host__ __device__ inline int mf_half(int nsb) { return nsb <= 4 ? nsb : min(nsb, ((nsb + 1) / 2 + 1) & ~1); }

template <bool GU, bool TL, int RT>
__global__ __launch_bounds__(256) void k_moe_mfma(int d, int ff, int n_act, const uint8_t *__restrict__ Wa,
                                                  const uint8_t *__restrict__ Wb, MoeWs ws)
{
    // RT (down projection only, with every super-block staged at once): a wave walks RT tiles of
    // 32 weight rows, 128 rows apart, one after the other on the same staged activations; the
    // weight loads run ahead across the tile boundaries.
    static_assert(RT == 1 || !GU, "row tiles in sequence: down projection only");
    // The chunk's activation bytes, staged per block in two halves (super-blocks 0 .. nh1-1, then
    // nh1 .. nsb-1, so that the LDS of a block is half the chunk's and more blocks fit a CU):
    // 1 KiB per sub-block c = 8 * sb + j, laid out [h][pair][16 B] so that the A operand of lane l
    // is the 16 bytes at l * 16.
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int s_pairs[MF_PCH];
    __shared__ float s_dx[16][MF_PCH];          // activation scale [super-block][chunk pair]
    __shared__ float s_up[GU ? 2 : 1][MF_PCH][33];
    const int u = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, col = lane & 31, h = lane >> 5;
    // One round trip for the chunk count, the chunk's expert and size, and its pair col (u <
    // gridDim.x keeps every index inside the workspace arrays; entries at or past the size are
    // stale and replaced by pair 0, which every chunk has).
    const int U = *ws.nuniq;
    const int ex = ws.uniq[u], cnt = ws.ucnt[u];
    int pc = ws.upairs[u * MF_PCH + col];
    if (u >= U) return;
    pc = __shfl(pc, col < cnt ? lane : 0, 64);
    if (t < MF_PCH) s_pairs[t] = pc;

    // Second round trip (weights, staged activations, activation scales), then one barrier.
    const int K = GU ? d : ff, nsb = K / 256, rec = q8k_rec_bytes(nsb);
    const uint8_t *X = GU ? ws.xrec : ws.xact;
    const int arow = GU ? pc / n_act : pc;          // activation row of pair col (the A row of lane l)
    for (int sb = 2 * w + h; sb < nsb; sb += 8)
        s_dx[sb][col] = ((const float *)(X + (size_t)arow * rec + nsb * 320))[sb];

    const int mat = GU ? (w & 1) : 0, nrows = GU ? ff : d;
    const int r0 = GU ? blockIdx.y * 64 + 32 * (w >> 1) : blockIdx.y * 128 * RT + 32 * w;
    const size_t erow = (size_t)nsb * 144;
    const uint8_t *wr = (mat ? Wb : Wa) + (size_t)ex * erow * nrows;
    // granule g of this lane's row in super-block sb: wr + wofs + sb * sbs + g * gs
    const size_t wofs = q4k_gofs<TL>((size_t)(r0 + col), 0, 0, nsb);
    constexpr int sbs = TL ? 1152 : 144, gs = TL ? 128 : 16;

    // Weight operands in a ring of NB register buffers: the loads run NB - 1 super-blocks ahead
    // of the math (the last ones reload the final super-block, in bounds).
    struct Wt {
        v4i hdr, q[4];
    };
    constexpr int NB = 2;
    Wt wb[NB];
    // step k: tile k / nsb (128 * tile rows further on, in both layouts), super-block k % nsb
    auto wload = [&](int k, Wt &o) {
        const int tile = RT > 1 ? k / nsb : 0, sb = k - tile * nsb;
        const uint8_t *b = wr + wofs + (size_t)tile * 128 * erow + sb * sbs;
        o.hdr = *(const v4i *)b;
#pragma unroll
        for (int p = 0; p < 4; p++) o.q[p] = *(const v4i *)(b + (1 + 2 * p + h) * gs);
    };
#pragma unroll
    for (int i = 0; i < NB - 1; i++) wload(min(i, nsb - 1), wb[i]);
    // DMA lane l fetches pair l % 32, bytes 16 * (l / 32) .. +16 of each sub-block.
    const uint8_t *src = X + (size_t)arow * rec + 16 * h;
    const int nh1 = mf_half(nsb);   // nsb, or even: the halves meet between two ring steps
    auto stage = [&](int sb0, int sb1) {
        for (int c = 8 * sb0 + w; c < 8 * sb1; c += 4) dma_1k(src + 32 * c, smem + (c - 8 * sb0) * 1024);
    };
    stage(0, nh1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();   // staged activations, s_dx, s_pairs

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    // Accumulator registers 4q .. 4q+3 hold chunk pairs 8q .. 8q+7: only the first nq quads hold
    // pairs of the chunk, so the scaling and the combine skip the others (a block-uniform branch).
    const int nq = (cnt + 7) / 8;
    // The 6-bit scale is folded into the weight operand: sc = sc_lo + 8 sc_hi with 3-bit halves, and
    // q * sc_lo, q * sc_hi <= 15 * 7 = 105 fit a signed byte, so two MFMAs per sub-block with
    // B = q * sc_lo and B = q * sc_hi accumulate sum_j sc_lo_j dot_j and sum_j sc_hi_j dot_j in
    // the matrix core, and isc = lo + 8 hi is the same integer as sum_j sc_j dot_j (no per-register
    // scale multiply-adds).  A lane's 16 weight bytes are one row and one sub-block, so one packed
    // 16-bit multiply per dword scales four bytes at once (each byte product stays below 256).
    auto compute = [&](int sb, const Wt &o) {
        const uint8_t *as = smem + (sb < nh1 ? sb : sb - nh1) * 8 * 1024 + lane * 16;
        int sc[8], mm[8];
        v16i lo = {}, hi = {}, imn = {};
        v4i a[9];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int m;
            gsm(o.hdr, j, sc[j], m);
            mm[j] = (int)__builtin_amdgcn_perm((uint32_t)m, (uint32_t)m, 0u);   // m in every byte
        }
        a[0] = *(const v4i *)as;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j < 7) a[j + 1] = *(const v4i *)(as + (j + 1) * 1024);
            const v4i b = (o.q[j >> 1] >> (4 * (j & 1))) & 0x0F0F0F0F;
            const u16x2 slo = u16x2{(uint16_t)(sc[j] & 7), (uint16_t)(sc[j] & 7)};
            const u16x2 shi = u16x2{(uint16_t)(sc[j] >> 3), (uint16_t)(sc[j] >> 3)};
            v4i blo, bhi;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int bv = b[t];   // bit-cast a scalar copy: clang's bit cast of a vector
                                       // element subscript reads element 0 whatever the index
                const u16x2 bt = __builtin_bit_cast(u16x2, bv);
                blo[t] = __builtin_bit_cast(int, bt * slo);
                bhi[t] = __builtin_bit_cast(int, bt * shi);
            }
            lo = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], blo, lo, 0, 0, 0);
            hi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], bhi, hi, 0, 0, 0);
            imn = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], v4i{mm[j], mm[j], mm[j], mm[j]}, imn, 0, 0, 0);
        }
#pragma unroll
        for (int qd = 0; qd < 4; qd++)
            if (qd < nq)
#pragma unroll
                for (int r = 4 * qd; r < 4 * qd + 4; r++) {
                    const int k = 8 * (r >> 2) + 4 * h + (r & 3);   // chunk pair of accumulator register r
                    acc[r] = acc[r] + q4k_combine(o.hdr, s_dx[sb][k], lo[r] + 8 * hi[r], imn[r]);
                }
    };
    const int nstep = RT * nsb;
    for (int k0 = 0; k0 < nstep; k0 += NB) {
        if (RT == 1 && k0 == nh1) {   // second half of the activations into the same LDS
            __syncthreads();
            stage(nh1, nsb);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int k = k0 + i;
            if (k < nstep) {
                wload(min(k + NB - 1, nstep - 1), wb[(i + NB - 1) % NB]);
                __builtin_amdgcn_sched_barrier(0);
                const int sb = RT > 1 ? k % nsb : k;
                compute(sb, wb[i]);
                if constexpr (RT > 1)
                    if (sb == nsb - 1 && k < nstep - 1) {   // a tile done: store it, start the next
                        const int rt = r0 + 128 * (k / nsb);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int kk = 8 * (r >> 2) + 4 * h + (r & 3);
                            if (kk < cnt) ws.ydn[(size_t)s_pairs[kk] * d + rt + col] = acc[r];
                            acc[r] = 0.0f;
                        }
                    }
            }
        }
    }

    if constexpr (GU) {
        if (mat == 1)
#pragma unroll
            for (int r = 0; r < 16; r++) s_up[w >> 1][8 * (r >> 2) + 4 * h + (r & 3)][col] = acc[r];
        __syncthreads();
        if (mat == 0)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int k = 8 * (r >> 2) + 4 * h + (r & 3);
                if (k < cnt) ws.act[(size_t)s_pairs[k] * ff + r0 + col] = swiglu(acc[r], s_up[w >> 1][k][col]);
            }
    } else {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int k = 8 * (r >> 2) + 4 * h + (r & 3);
            if (k < cnt) ws.ydn[(size_t)s_pairs[k] * d + r0 + 128 * (RT - 1) + col] = acc[r];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// grid (U_max, d / DN_ROWS).  Units (row, super-block) = DN_ROWS*nsf, 8 lanes each.
// ------------------------------------------------------------------------------------------------
template <int UPL, bool TL>
__global__ __launch_bounds__(256) void k_moe_down(int d, int ff, const uint8_t *__restrict__ Wd, MoeWs ws)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int u = blockIdx.x;
    // Union slot metadata in one round trip (entries of slots >= U are stale and unused).
    const int U = *ws.nuniq;
    const int ex = ws.uniq[u], cnt = ws.ucnt[u];
    const int prl = ws.upairs[u * 8 + (threadIdx.x & 7)];   // lane l holds pair l % 8 of the slot
    if (u >= U) return;
    const int lane = threadIdx.x & 63, w = wave_id(), i = lane & 7;
    const int nsf = ff / 256;
    const int r0 = blockIdx.y * DN_ROWS;
    const int nunits = DN_ROWS * nsf;
    const size_t erow = (size_t)nsf * 144;
    const size_t emat = erow * d;

    v4i hdr[UPL], qs[UPL];
#pragma unroll
    for (int c = 0; c < UPL; c++) {
        const int un = min(c * 32 + w * 8 + (lane >> 3), nunits - 1);   // clamped, as in gate/up
        const int r = un / nsf, sb = un - r * nsf;
        const uint8_t *wm = Wd + (size_t)ex * emat;
        hdr[c] = *(const v4i *)(wm + q4k_gofs<TL>((size_t)(r0 + r), sb, 0, nsf));
        qs[c] = __builtin_nontemporal_load((const v4i *)(wm + q4k_gofs<TL>((size_t)(r0 + r), sb, 1 + i, nsf)));
    }

    // Q8_K of this expert's activation rows (one wave per 256-element block) -> LDS.
    int8_t *aq = (int8_t *)smem;                    // [8][nsf][256]
    int *abs_ = (int *)(aq + 8 * nsf * 256);        // [8][nsf][16]
    float *ad = (float *)(abs_ + 8 * nsf * 16);     // [8][nsf]
    float *tv = ad + 8 * nsf;                       // [8][DN_ROWS][nsf]
    // 16 blocks per pass (4 per wave), each pass's loads issued before its math; the first pass is
    // straight-line code so that its loads go out right behind the weight loads.
    const int nq = cnt * nsf;
    float4 v[4];
#define X100_ACT_LOADS(q0)                                                                        \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                               \
        const int q = min((q0) + 4 * j + w, nq - 1); /* clamped; only q < nq is used */           \
        const int k = q / nsf, sb = q - k * nsf;                                                  \
        v[j] = *(const float4 *)(ws.act + (size_t)__builtin_amdgcn_readlane(prl, k) * ff + sb * 256 + 4 * lane); \
    }
#define X100_ACT_QUANT(q0)                                                                        \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                               \
        const int q = (q0) + 4 * j + w;                                                           \
        if (q < nq) q8_K_wave(v[j], aq + q * 256, abs_ + q * 16, ad + q);                          \
    }
    X100_ACT_LOADS(0)
    __builtin_amdgcn_sched_barrier(0);
    X100_ACT_QUANT(0)
    for (int q0 = 16; q0 < nq; q0 += 16) {
        X100_ACT_LOADS(q0)
        X100_ACT_QUANT(q0)
    }
#undef X100_ACT_LOADS
#undef X100_ACT_QUANT
    __shared__ int s_pr[8];
    if (threadIdx.x < 8) s_pr[threadIdx.x] = prl;
    __syncthreads();

    // As in gate/up: pairs outer, units inner, branch-free (spare slot 8 * nunits).
    for (int k = 0; k < cnt; k++) {
#pragma unroll
        for (int c = 0; c < UPL; c++) {
            const int un = c * 32 + w * 8 + (lane >> 3);
            const bool valid = un < nunits;
            const int sb = valid ? un % nsf : 0;
            int isc, imn;
            q4k_unit_dot(hdr[c], qs[c], aq + (k * nsf + sb) * 256, abs_ + (k * nsf + sb) * 16, i, isc, imn);
            tv[valid ? k * nunits + un : 8 * nunits] = q4k_combine(hdr[c], ad[k * nsf + sb], isc, imn);
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < cnt * DN_ROWS; t += 256) {
        const int k = t / DN_ROWS, r = t - k * DN_ROWS;
        float y = 0.0f;
        for (int sb = 0; sb < nsf; sb++) y = y + tv[k * nunits + r * nsf + sb];
        ws.ydn[(size_t)s_pr[k] * d + r0 + r] = y;
    }
}

// ------------------------------------------------------------------------------------------------
// Down projection and weighted combine in one launch.  grid (d / DN, row groups of rg token rows);
// a block owns DN output rows for every (token row m, slot a) pair p = m*n_act + a of its row group
// (at most 32 pairs; the pairs below are the group's).  Units (pair p, row r, super-block
// sb) = P*DN*nsf in that order, two lanes each (halves of the Q4_K block), UPL units per lane
// pair: the unit's expert is sel[p] and its activation row is act[p] (an expert chosen by several
// token rows is read once per pair, the repeats mostly from cache), so the activation loads depend
// on nothing and the weight loads only on sel.  The block's waves quantize the P*nsf activation
// records (Q8_K) into LDS, four per pass; y(p, r) sums the super-blocks in order and
// out[m][r] (+)= sum over slots a = 0..n_act-1 of w_a * y (qwen_moe.c:310-311), as k_moe_down and
// k_moe_combine do.
// ------------------------------------------------------------------------------------------------
constexpr int FD_DN = 8;     // output rows per block

// Wait until at most n of this wave's vector memory operations are outstanding (n wave-uniform;
// above 15 it waits for all of them, which is never too early).
X100_DEV void vm_wait_upto(int n)
{
    switch (__builtin_amdgcn_readfirstlane(n)) {
#define X100_VMW(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        X100_VMW(1) X100_VMW(2) X100_VMW(3) X100_VMW(4) X100_VMW(5) X100_VMW(6) X100_VMW(7) X100_VMW(8)
        X100_VMW(9) X100_VMW(10) X100_VMW(11) X100_VMW(12) X100_VMW(13) X100_VMW(14) X100_VMW(15)
#undef X100_VMW
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

template <int UPL, bool TL>
__global__ __launch_bounds__(1024) void k_moe_down_fused(int M, int rg, int d, int ff, int n_exp, int n_act, uint32_t mnsf,
                                                        uint32_t mdn, uint32_t mspan, const uint8_t *__restrict__ Wd, MoeWs ws,
                                                        float *__restrict__ out, int residual,
                                                        const float *__restrict__ oadd)
{
    constexpr int DN = FD_DN;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float s_y[32][FD_DN];
    __shared__ float s_w[32];
    const int lane = threadIdx.x & 63, w = wave_id(), h = lane & 1, nw = blockDim.x >> 6;
    const int m0 = blockIdx.y * rg, Mg = min(rg, M - m0);   // the group's token rows
    const int P = Mg * n_act, p0 = m0 * n_act;               // its pairs: p0 .. p0 + P - 1
    const int nsf = ff / 256;
    const int r0 = blockIdx.x * DN;
    const int nunits = P * DN * nsf, nq = P * nsf;
    const size_t erow = (size_t)nsf * 144;
    const size_t emat = erow * d;
    uint8_t *recs = smem;                              // [nq][KREC] activation records
    uint8_t *wl = smem + (size_t)nq * KREC;            // [nunits][144] weight blocks (padded to KiB)
    float *tv = (float *)(wl + ((size_t)nunits * 9 + 63) / 64 * 1024);   // [P][DN][nsf] + one spare

    // Waves 0 .. nwq-1 quantize the activation records (four per pass); the others stage the weight
    // blocks, so the two run side by side.  The units of pair p are rows r0 .. r0+DN-1 of expert
    // sel[p], one contiguous span of DN * erow bytes: DMA op i copies 16-byte chunks 64i .. 64i+63
    // of the P spans in pair order (chunks past the end clamped onto the last one, the LDS area
    // padded to whole KiB), so LDS holds the units' blocks in unit order (144 bytes each).
    // (One wave does both.)
    const int nwq = nw / 2;
    if (w < nwq || nw == 1) {
        // The activation rows were written by the previous launch, so every load is a round trip
        // to memory: the loads of four passes are issued before the first is quantized (passes past
        // the last record read out of range, which returns zeros and touches no memory).
        const rsrc_t ar = buf_rsrc(ws.act + (size_t)p0 * ff, (uint32_t)(P * ff) * 4u);
        const int step = 4 * max(nwq, 1);
        for (int qb0 = 4 * w; qb0 < nq; qb0 += 4 * step) {
            float4 v[4][4];
#pragma unroll
            for (int p = 0; p < 4; p++) q8k_load(ar, ff, nsf, mnsf, nq, qb0 + p * step, v[p]);
#pragma unroll
            for (int p = 0; p < 4; p++)
                if (qb0 + p * step < nq) q8k_quant(v[p], nq, qb0 + p * step, recs);
        }
    }
    // With two unit slots per lane (UPL = 2) the dots run in two phases: slot 0 of every wave
    // computes as soon as the DMA operations of the pairs it reads have landed, while the later
    // operations are still in flight, then slot 1 (M = 4: 27.2 -> 26.7 us per layer).  For that the
    // weight DMA is issued from inline asm (dma16v, not counted by the compiler), in ascending order
    // per wave, and each DMA wave waits for its early operations with an exact vmcnt.  With one slot
    // per lane the compiler-counted DMA and a single barrier are faster (the asm issue alone cost
    // 0.3 us at M = 1).
    constexpr bool SPLIT = UPL == 2;
    const int nch = nunits * 9, span = DN * nsf * 9;   // 16-byte chunks: total, per pair
    const int nops = (nch + 63) / 64, ndw = nw - nwq;
    const int pa = min(P, (32 * nw + DN * nsf - 1) / (DN * nsf));   // pairs that slot 0 reads
    const int I1 = min(nops, (pa * span + 63) / 64);                // operations those pairs need
    int nlate = 0;
    if (w >= nwq) {
        const int selv = (int)min((unsigned)ws.sel[p0 + min(lane, P - 1)], (unsigned)(n_exp - 1));
        const int j = w - nwq;
        for (int i = j; i < nops; i += ndw) {
            const int c = min(i * 64 + lane, nch - 1);
            const int p = (int)udiv16((uint32_t)c, (uint32_t)span, mspan);
            const int ex = __shfl(selv, p, 64);
            const uint8_t *src = Wd + (size_t)ex * emat + (size_t)r0 * erow + 16 * (size_t)(c - p * span);
            if constexpr (SPLIT)
                dma16v(src, __builtin_amdgcn_readfirstlane(lds_addr(wl) + (uint32_t)i * 1024u));
            else
                dma_1k(src, wl + i * 1024);
        }
        if constexpr (SPLIT) {
            const int i0 = j >= I1 ? j : j + (I1 - j + ndw - 1) / ndw * ndw;   // first late operation
            nlate = i0 < nops ? (nops - 1 - i0) / ndw + 1 : 0;
        }
    }
    if ((int)threadIdx.x < P) s_w[threadIdx.x] = ws.sw[p0 + threadIdx.x];
    if constexpr (SPLIT) {
        vm_wait_upto(nlate);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        __syncthreads();
    }

    // the units of slot c
    auto slot = [&](int c) __attribute__((always_inline)) {
        // unit un = (pair, row, super-block) in that order; tiled, the lanes take the units
        // row-fastest (q = (pair, super-block, row)), so that 8 consecutive lane pairs read the 8
        // rows (DN = 8) of one LDS tile
        const int q = c * 32 * nw + w * 32 + (lane >> 1);
        const bool valid = q < nunits;
        const int qc = valid ? q : 0;
        const int p = (int)udiv16((uint32_t)qc, (uint32_t)(DN * nsf), mdn), rem = qc - p * DN * nsf;
        int un, sb;
        const uint8_t *blk;
        if constexpr (TL) {
            static_assert(DN == 8, "a tiled span holds 8 rows");
            sb = rem >> 3;
            un = (p * DN + (rem & 7)) * nsf + sb;
            blk = wl + (size_t)p * DN * nsf * 144 + sb * 1152 + 16 * (rem & 7);
        } else {
            un = qc;
            sb = rem - (int)udiv16((uint32_t)rem, (uint32_t)nsf, mnsf) * nsf;
            blk = wl + (size_t)qc * 144;
        }
        v4i hdr, qv[4];
        q4k_lds_unit<TL>(blk, h, hdr, qv);
        Q4kHalf uh;
        q4k_scales_gguf(hdr, h, uh);
        q4k_unpack(qv, uh);
        const uint32_t h0 = (uint32_t)hdr[0];
        const uint8_t *rec = recs + (size_t)(p * nsf + sb) * KREC;
        int isc, imn;
        q4k_half_sums(uh, rec, h, isc, imn);
        tv[valid ? un : nunits] = q4k_term(h2f((uint16_t)(h0 & 0xffff)), h2f((uint16_t)(h0 >> 16)),
                                           *(const float *)(rec + KR_D), isc, imn);
    };
    if constexpr (SPLIT) {
        slot(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the late operations
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        slot(1);
    } else {
#pragma unroll
        for (int c = 0; c < UPL; c++) slot(c);
    }
    __syncthreads();
    // y of each (pair, row): sequential over super-blocks (the oracle's order)
    for (int t = threadIdx.x; t < P * DN; t += blockDim.x) {
        const int p = t / DN, r = t - p * DN;
        float y = 0.0f;
        for (int sb = 0; sb < nsf; sb++) y = y + tv[(p * DN + r) * nsf + sb];
        s_y[p][r] = y;
    }
    __syncthreads();
    // out[m][row] (+)= sum over slots a of w_a * y_a, a ascending (qwen_moe.c:310-311)
    for (int t = threadIdx.x; t < Mg * DN; t += blockDim.x) {
        const int m = t / DN, r = t - m * DN;
        float eo = 0.0f;
        for (int a = 0; a < n_act; a++) eo = eo + s_w[m * n_act + a] * s_y[m * n_act + a][r];
        const size_t i = (size_t)(m0 + m) * d + r0 + r;
        out[i] = residual ? (oadd ? out[i] + oadd[i] : out[i]) + eo : eo;
    }
}

// ------------------------------------------------------------------------------------------------
// out[m][j] (+)= sum_a sw[m][a] * y[m*n_act + a][j], a ascending (qwen_moe.c:310-311).  With oadd
// (the decoder layer's attention output, whose residual add a folded router left undone) the
// residual is (out + oadd) + the sum, the order of the unfolded layer.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_moe_combine(int M, int d, int n_act, MoeWs ws,
                                                     float *__restrict__ out, int residual,
                                                     const float *__restrict__ oadd)
{
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= M * d) return;
    const int m = t / d, j = t - m * d;
    float wv[8], yv[8];
#pragma unroll
    for (int a = 0; a < 8; a++)
        if (a < n_act) {
            wv[a] = ws.sw[m * n_act + a];
            yv[a] = ws.ydn[(size_t)(m * n_act + a) * d + j];
        }
    float eo = 0.0f;
#pragma unroll
    for (int a = 0; a < 8; a++)
        if (a < n_act) eo = eo + wv[a] * yv[a];
    out[t] = residual ? (oadd ? out[t] + oadd[t] : out[t]) + eo : eo;
}

MoeWs carve(uintptr_t base, int M, int d, int ff, int n_exp, int n_act, size_t *total)
{
    const int P = M * n_act;
    const int nsb = d / 256;
    size_t off = 0;
    MoeWs ws;
    auto take = [&](size_t bytes) {
        void *r = (void *)(base + off);
        off += al(bytes);
        return r;
    };
    ws.logits = (float *)take(sizeof(float) * M * n_exp);
    ws.sel = (int *)take(sizeof(int) * P);
    ws.sw = (float *)take(sizeof(float) * P);
    ws.nuniq = (int *)take(sizeof(int));
    ws.uniq = (int *)take(sizeof(int) * P);
    ws.ucnt = (int *)take(sizeof(int) * P);
    // union slots of 8 (up to 8 rows: at most P of them) or chunks of 32 (at most P/32 + n_exp + 1, and
    // at most P)
    ws.upairs = (int *)take(sizeof(int) * ((size_t)P * 8 + 32 * (size_t)n_exp + 32));
    // hn records: Q8_K records [M][nsb] (up to 8 rows) or per-row records (the matrix-core path)
    ws.xrec = (uint8_t *)take(max((size_t)M * q8k_rec_bytes(nsb), (size_t)M * nsb * KREC));
    ws.act = (float *)take(sizeof(float) * (size_t)P * ff);
    ws.ydn = (float *)take(sizeof(float) * (size_t)P * d);
    ws.xact = (uint8_t *)take((size_t)P * q8k_rec_bytes(ff / 256));
    if (total) *total = off;
    return ws;
}

void route_rows(int M, int d, int n_exp, const float *hn, const float *R, MoeWs ws, hipStream_t s)
{
    const int epw = max(1, min(8, M / 64));   // experts per wave
    const int ngrp = (n_exp + 4 * epw - 1) / (4 * epw), nq = (RR_ROWS * (d / 256) + 3) / 4;
    const dim3 g(ngrp + nq, (M + RR_ROWS - 1) / RR_ROWS);
    if (d == 2048)
        hipLaunchKernelGGL((k_moe_route_rows<8, true>), g, dim3(256), 0, s, M, d, n_exp, epw, hn, R, ws);
    else if (d < 2048)
        hipLaunchKernelGGL((k_moe_route_rows<8, false>), g, dim3(256), 0, s, M, d, n_exp, epw, hn, R, ws);
    else if (d == 4096)
        hipLaunchKernelGGL((k_moe_route_rows<16, true>), g, dim3(256), 0, s, M, d, n_exp, epw, hn, R, ws);
    else
        hipLaunchKernelGGL((k_moe_route_rows<16, false>), g, dim3(256), 0, s, M, d, n_exp, epw, hn, R, ws);
}

// Nine or more token rows, on the matrix cores: router logits and Q8_K records per 4-row chunk,
// softmax / top-k per 8-row chunk, the pairs grouped by expert into chunks of 32, gate/up + SwiGLU
// and the down projection by k_moe_mfma, then the weighted combine.
template <bool TL>
hipError_t moe_launch_mfma(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                           const void *Wg, const void *Wu, const void *Wd, float *out, int residual, int *sel,
                           float *sw, MoeWs ws, hipStream_t s)
{
    const int nsb = d / 256, nsf = ff / 256, P = M * n_act, nrc = (M + 7) / 8;
    const int Vmax = min(P, (P + MF_PCH - 1) / MF_PCH + n_exp);
    route_rows(M, d, n_exp, hn, R, ws, s);
    hipLaunchKernelGGL(k_moe_topk_rows, dim3(nrc), dim3(512), 0, s, M, n_exp, n_act, ws, sel, sw);
    hipLaunchKernelGGL(k_moe_group<MF_PCH>, dim3(1), dim3(256), 0, s, P, n_exp, ws);
    hipLaunchKernelGGL((k_moe_mfma<true, TL, 1>), dim3(Vmax, ff / 64), dim3(256), (size_t)mf_half(nsb) * 8192, s, d,
                       ff, n_act, (const uint8_t *)Wg, (const uint8_t *)Wu, ws);
    hipLaunchKernelGGL(k_moe_act_q8k, dim3((P * nsf + 3) / 4), dim3(256), 0, s, P, ff, ws);
    // down: MF_DN_RT row tiles per wave when one staging part holds every super-block
    if (MF_DN_RT > 1 && mf_half(nsf) == nsf && d % (128 * MF_DN_RT) == 0)
        hipLaunchKernelGGL((k_moe_mfma<false, TL, MF_DN_RT>), dim3(Vmax, d / (128 * MF_DN_RT)), dim3(256),
                           (size_t)nsf * 8192, s, d, ff, n_act, (const uint8_t *)Wd, (const uint8_t *)nullptr, ws);
    else
        hipLaunchKernelGGL((k_moe_mfma<false, TL, 1>), dim3(Vmax, d / 128), dim3(256), (size_t)mf_half(nsf) * 8192, s, d,
                           ff, n_act, (const uint8_t *)Wd, (const uint8_t *)nullptr, ws);
    hipLaunchKernelGGL(k_moe_combine, dim3((M * d + 255) / 256), dim3(256), 0, s, M, d, n_act, ws, out, residual,
                       (const float *)nullptr);
    return hipGetLastError();
}

// Below MF_MIN_ROWS token rows: routing, gate/up (persistent), down (+ combine).  With nrm (one
// row, d = 2048), hn is the layer's h: the router forms rmsnorm(h + oadd, nrm) itself
// (k_moe_route_norm) and the residual output is (h + oadd) + the MoE sum.
template <bool TL>
hipError_t moe_launch_few(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                          const void *Wg, const void *Wu, const void *Wd, float *out, int residual, int *sel,
                          float *sw, MoeWs ws, hipStream_t s, const float *oadd = nullptr,
                          const float *nrm = nullptr, float eps = 0.0f)
{
    const int nsb = d / 256, nsf = ff / 256;
    const int Umax = min(M * n_act, n_exp);

    const int nwaves = n_exp * M + (M * nsb + 3) / 4;   // router waves, then quantizer waves of four records
    if (nrm)
        hipLaunchKernelGGL(k_moe_route_norm, dim3((nwaves + RT_WPB - 1) / RT_WPB), dim3(64 * RT_WPB), 0, s, n_exp,
                           hn, oadd, nrm, eps, R, ws);
    else
        hipLaunchKernelGGL(k_moe_route, dim3((nwaves + RT_WPB - 1) / RT_WPB), dim3(64 * RT_WPB),
                           (size_t)min(M, RT_WPB) * d * 4, s, M, d, n_exp, udiv16_magic((uint32_t)nsb), hn, R, ws);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;

    // Gate/up (k_moe_gate_up_p): as many persistent blocks as are resident at once, at most one per
    // work item, each deriving the routing itself (cheaper than a separate routing launch) and
    // holding two weight buffers.
    const uint8_t *wg = (const uint8_t *)Wg, *wu = (const uint8_t *)Wu;
    const size_t lds_gp = ((size_t)M * nsb * KREC + 1023) / 1024 * 1024 +                // hn records
                          2 * (((size_t)2 * GU_ROWS * nsb * 9 + 63) / 64 * 1024) +       // weight blocks x 2
                          ((size_t)M * 2 * GU_ROWS * nsb + 1) * 4 +                       // terms
                          (size_t)Umax * 9 * 4;                                           // slot lists
    const int upl_gu = (2 * 2 * GU_ROWS * nsb + 64 * GU_NWV - 1) / (64 * GU_NWV);   // two lanes per unit
#define X100_GU(U)                                                                                       \
    do {                                                                                                 \
        const int nb = min(Umax * (ff / GU_ROWS), resident_blocks(k_moe_gate_up_p<U, GU_NWV, TL>, 64 * GU_NWV, lds_gp)); \
        hipLaunchKernelGGL((k_moe_gate_up_p<U, GU_NWV, TL>), dim3(nb), dim3(64 * GU_NWV), lds_gp, s, M, d, ff, n_exp, \
                           n_act, wg, wu, ws, sel, sw);                                                   \
    } while (0)
    if (upl_gu == 1)
        X100_GU(1);
    else
        X100_GU(2);   // at most 2 * GU_ROWS * 16 units (d <= 4096)
#undef X100_GU
    err = hipGetLastError();
    if (err != hipSuccess) return err;

    {
        // down + combine in one launch (k_moe_down_fused) when the units fit two per lane pair in
        // 16 waves and the activation records fit LDS (every block quantizes all pairs of its row
        // group); otherwise k_moe_down, then k_moe_combine.  Row groups: the fewest groups of at
        // most 32 pairs, rows spread evenly over them (8 rows of 8 slots: two groups of 4).
        const int dn = FD_DN;
        const int ng = (M * n_act + 31) / 32, rg = (M + ng - 1) / ng;
        const int P = rg * n_act, nq = P * nsf, nun = P * dn * nsf;
        const int upl = (2 * nun + 1023) / 1024;
        const int nwf = (2 * nun + 64 * upl - 1) / (64 * upl);
        const size_t ldsf = (size_t)nq * KREC + ((size_t)nun * 9 + 63) / 64 * 1024 + ((size_t)nun + 1) * 4;
        if (P <= 32 && d % dn == 0 && upl <= 2 && ldsf <= 160 * 1024) {
            const dim3 gf(d / dn, (M + rg - 1) / rg), bf(64 * nwf);
            const uint32_t mnsf = udiv16_magic((uint32_t)nsf), mdn = udiv16_magic((uint32_t)(dn * nsf));
            const uint32_t mspan = udiv16_magic((uint32_t)(dn * nsf * 9));
            if (upl == 1)
                hipLaunchKernelGGL((k_moe_down_fused<1, TL>), gf, bf, ldsf, s, M, rg, d, ff, n_exp, n_act, mnsf, mdn,
                                   mspan, (const uint8_t *)Wd, ws, out, residual, oadd);
            else
                hipLaunchKernelGGL((k_moe_down_fused<2, TL>), gf, bf, ldsf, s, M, rg, d, ff, n_exp, n_act, mnsf, mdn,
                                   mspan, (const uint8_t *)Wd, ws, out, residual, oadd);
            return hipGetLastError();
        }
    }
    const size_t lds_dn = (size_t)8 * nsf * (256 + 64 + 4) + ((size_t)8 * DN_ROWS * nsf + 1) * 4;
    const int upl_dn = (DN_ROWS * nsf + 31) / 32;
    const dim3 g_dn(Umax, d / DN_ROWS);
    const uint8_t *wd = (const uint8_t *)Wd;
    switch (upl_dn) {
    case 1: hipLaunchKernelGGL((k_moe_down<1, TL>), g_dn, dim3(256), lds_dn, s, d, ff, wd, ws); break;
    case 2: hipLaunchKernelGGL((k_moe_down<2, TL>), g_dn, dim3(256), lds_dn, s, d, ff, wd, ws); break;
    case 3: case 4: hipLaunchKernelGGL((k_moe_down<4, TL>), g_dn, dim3(256), lds_dn, s, d, ff, wd, ws); break;
    default: hipLaunchKernelGGL((k_moe_down<8, TL>), g_dn, dim3(256), lds_dn, s, d, ff, wd, ws); break;
    }
    err = hipGetLastError();
    if (err != hipSuccess) return err;

    hipLaunchKernelGGL(k_moe_combine, dim3((M * d + 255) / 256), dim3(256), 0, s, M, d, n_act, ws, out, residual, oadd);
    return hipGetLastError();
}

// Tiled expert layout (q4k_gofs<true>): thread t writes 16-byte granule t of dst, whose tile
// position (row group, super-block, granule, row) names the granule of src it copies.
__global__ __launch_bounds__(256) void k_moe_tile_pack(size_t ngran, int nsb, const v4i *__restrict__ src,
                                                       v4i *__restrict__ dst)
{
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= ngran) return;
    const size_t tile = t / 72;   // 8 rows x 9 granules
    const int in = (int)(t - tile * 72), g = in >> 3, r7 = in & 7;
    const size_t rg = tile / nsb;
    const int sb = (int)(tile - rg * nsb);
    dst[t] = src[((8 * rg + r7) * nsb + sb) * 9 + g];
}

}  // namespace

size_t x100_moe_workspace_bytes(int M, int d, int ff, int n_exp, int n_act)
{
    size_t total = 0;
    carve(0, M, d, ff, n_exp, n_act, &total);
    return total;
}

static bool moe_shape_ok(int M, int d, int ff, int n_exp, int n_act, int flags)
{
    if (M < 1 || M > X100_MOE_MAX_ROWS || n_act < 1 || n_act > 8 || n_exp < n_act || n_exp > 256) return false;
    if (d % 256 || ff % 256 || d > 4096 || ff > 4096 || d % DN_ROWS || ff % GU_ROWS) return false;
    if (flags & ~(X100_MOE_RESIDUAL | X100_MOE_TILED)) return false;
    return 2 * GU_ROWS * (d / 256) <= 8 * 8 * GU_NWV && DN_ROWS * (ff / 256) <= 8 * 32;
}

bool x100_moe_norm_supported(int d, int ff, int n_exp, int n_act, int flags)
{
    return d == 2048 && flags == X100_MOE_RESIDUAL && moe_shape_ok(1, d, ff, n_exp, n_act, flags);
}

hipError_t x100_moe_norm_launch(int d, int ff, int n_exp, int n_act, float *h, const float *o, const float *nrm,
                                float eps, const float *R, const void *Wg, const void *Wu, const void *Wd, int flags,
                                int *sel, float *sw, void *workspace, hipStream_t s)
{
    if (!x100_moe_norm_supported(d, ff, n_exp, n_act, flags) || !o || !nrm) return hipErrorInvalidValue;
    MoeWs ws = carve((uintptr_t)workspace, 1, d, ff, n_exp, n_act, nullptr);
    return moe_launch_few<false>(1, d, ff, n_exp, n_act, h, R, Wg, Wu, Wd, h, 1, sel, sw, ws, s, o, nrm, eps);
}

hipError_t x100_moe_launch(int M, int d, int ff, int n_exp, int n_act, const float *hn, const float *R,
                           const void *Wg, const void *Wu, const void *Wd, float *out, int flags,
                           int *sel, float *sw, void *workspace, hipStream_t s)
{
    if (!moe_shape_ok(M, d, ff, n_exp, n_act, flags)) return hipErrorInvalidValue;
    MoeWs ws = carve((uintptr_t)workspace, M, d, ff, n_exp, n_act, nullptr);
    const int residual = flags & X100_MOE_RESIDUAL;
    const bool tiled = (flags & X100_MOE_TILED) != 0;
    if (M >= MF_MIN_ROWS)
        return tiled ? moe_launch_mfma<true>(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, s)
                     : moe_launch_mfma<false>(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, s);
    return tiled ? moe_launch_few<true>(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, s)
                 : moe_launch_few<false>(M, d, ff, n_exp, n_act, hn, R, Wg, Wu, Wd, out, residual, sel, sw, ws, s);
}

hipError_t x100_moe_tile_pack(int n_exp, int rows, int K, const void *src, void *dst, hipStream_t s)
{
    if (n_exp < 1 || rows < 8 || rows % 8 || K < 256 || K % 256 || !src || !dst) return hipErrorInvalidValue;
    const size_t ngran = (size_t)n_exp * rows * (K / 256) * 9;
    hipLaunchKernelGGL(k_moe_tile_pack, dim3((unsigned)((ngran + 255) / 256)), dim3(256), 0, s, ngran, K / 256,
                       (const v4i *)src, (v4i *)dst);
    return hipGetLastError();
}
