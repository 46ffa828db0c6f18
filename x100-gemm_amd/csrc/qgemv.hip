// Block-quantized dequant-GEMV for gfx950:  y[M][N] = W[N][K] . x[M][K]^T,  M <= 8.
//
// Weights are block-quantized (Q4_0, Q4_K, Q3_K, and Q8_0 / Q5_K / Q6_K through the int8 path);
// each x row is quantized inside the kernel (Q8_0 for Q4_0, Q8_K for the K-quants, Q8_0 with an
// fp32 scale for the int8 path) with the same fp32 operations as the scalar path
// (quantize_q8_0_native, qwen_moe_hp.c:408-414; pack_A_q3k, qwen_moe_q3k.c:612-624; pack_A_i8,
// qwen_moe_q3k.c:420-427), then every block's dot product is done in exact integer arithmetic
// with v_dot4 and scaled in fp32.
//
// At M <= 8 the work is bandwidth bound: every lane issues all of its 16-byte weight loads before
// it quantizes x, so a block's whole weight slice is in flight at once; no MFMA.
//
// Device weight layouts (made once at upload by x100q_pack):
//   Q4_K  GGUF-native 144-byte blocks (16-byte aligned fields, consumed as is).
//   Q4_0  split into d[N*K/32] (fp16) and qs[N*K/32][16], so nibble rows are 16-byte aligned.
//   Q3_K  split into hq[N*K/256][96] (hmask 32 + qs 64), sc[N*K/256][12], d[N*K/256] (fp16).
//   Q8_0, Q5_K, Q6_K  requantized to Q8_0 (the reference loader's lin_new_i8) and split into
//         d[N*K/32] (fp16) and qs[N*K/32][32].
// Q4_0 / Q4_K / Q3_K keep the GGUF blocks' byte count (plus alignment padding between the
// arrays); the int8 path stores 34 bytes per 32 elements.
//
// The K-quant kernels reduce each row in the same order as the scalar oracle (sequential over
// super-blocks, no fused multiply-add), so their fp32 outputs are bit-identical to it; Q4_0 sums
// lane partials in a tree (fp32 reassociation only).
#include "x100_common.h"
#include "x100_internal.h"

namespace {

// get_scale_min_k4 (repack.cpp:222-233) on the 12 scale bytes held in dwords s0, s1, s2.
X100_DEV uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int k)
{
    const uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
    return (w >> (8 * (k & 3))) & 0xffu;
}
X100_DEV void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m)
{
    // Both forms computed and selected (j is lane-dependent here: a branch would split the
    // unrolled loop); byte indices are taken modulo 12 so every read stays in the 12 bytes.
    const uint32_t bj = sbyte(s0, s1, s2, j), bj4 = sbyte(s0, s1, s2, (j + 4) % 12);
    const uint32_t bjm4 = sbyte(s0, s1, s2, (j + 8) % 12);   // byte j - 4 for j >= 4
    const int sc_lo = (int)(bj & 63), m_lo = (int)(bj4 & 63);
    const int sc_hi = (int)((bj4 & 0xf) | ((bjm4 >> 6) << 4));
    const int m_hi = (int)((bj4 >> 4) | ((bj >> 6) << 4));
    sc = j < 4 ? sc_lo : sc_hi;
    m = j < 4 ? m_lo : m_hi;
}

// ------------------------------------------------------------------------------------------------
// Q4_0 x Q8_0
// ------------------------------------------------------------------------------------------------
// Block = NT/64 waves; wave w owns rows row0 + w*RPW .. +RPW-1; lane l owns blocks l, l+64, ...
// (BPL per row).  All RPW*BPL nibble loads (16 B) and scale loads are issued first.
template <int MR, int RPW, int BPL, int XPT, int NT>
__global__ __launch_bounds__(NT) void k_q4_0(int M, int N, int K, const uint16_t *__restrict__ wd,
                                              const uint8_t *__restrict__ wq,
                                              const float *__restrict__ x, float *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / 32;
    const int nb1 = MR * nb + 1;                 // + the quantizer's spare block
    int8_t *xlo = (int8_t *)smem;
    int8_t *xhi = xlo + nb1 * 16;
    float *xd = (float *)(xhi + nb1 * 16);
    int *xs = (int *)(xd + nb1);

    const int lane = threadIdx.x & 63, w = wave_id();
    const int rowb = blockIdx.x * (NT / 64) * RPW + w * RPW;

    const int total4 = M * K / 4;
    const rsrc_t xr = buf_rsrc(x, (uint32_t)total4 * 16u);
    float4 xv[XPT];
    x_load<XPT, NT>(xr, 0, xv);

    // Unconditional loads (indices clamped into the matrix; out-of-range results are discarded),
    // so every load of the lane is in flight before the first one is waited for.
    v4i q[RPW][BPL];
    uint32_t dwb[RPW][BPL];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            const int row = min(rowb + r, N - 1), b = min(lane + 64 * c, nb - 1);
            const size_t blk = (size_t)row * nb + b;
            q[r][c] = __builtin_nontemporal_load((const v4i *)(wq + blk * 16));
            dwb[r][c] = wd[blk];
        }

    __builtin_amdgcn_sched_barrier(0);   // keep every load above ahead of the quantizer's math
    q8_0_from_regs<XPT, NT>(xv, 0, total4, K, xlo, xhi, xd, xs);
    for (int c0 = NT * XPT; c0 < total4; c0 += NT * XPT) {
        x_load<XPT, NT>(xr, c0, xv);
        q8_0_from_regs<XPT, NT>(xv, c0, total4, K, xlo, xhi, xd, xs);
    }
    __syncthreads();

#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int row = rowb + r;
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) acc[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            // Branch-free (the scheduler interleaves the unrolled blocks): a lane past the last
            // block reads block nb-1 and adds 0.  Rows m >= M compute on unused LDS and are not
            // stored.
            const bool inb = lane + 64 * c < nb;
            const int b = min(lane + 64 * c, nb - 1);
            const v4i qq = q[r][c];
            const float dwf = h2f((uint16_t)dwb[r][c]);
            int lo[4], hi[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                lo[t] = qq[t] & 0x0F0F0F0F;
                hi[t] = (qq[t] >> 4) & 0x0F0F0F0F;
            }
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const v4i xl = *(const v4i *)(xlo + (m * nb + b) * 16);
                const v4i xh = *(const v4i *)(xhi + (m * nb + b) * 16);
                int s = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    s = dot4(lo[t], xl[t], s);
                    s = dot4(hi[t], xh[t], s);
                }
                s -= 8 * xs[m * nb + b];  // nibble offset: (q-8).x = q.x - 8*sum(x)
                const float term = (float)s * (dwf * xd[m * nb + b]);
                acc[m] += inb ? term : 0.0f;
            }
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (m < M) {
                const float v = wave_sum_uf(acc[m]);
                if (lane == 0 && row < N) y[(size_t)m * N + row] = v;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// K-quants (Q4_K, Q3_K) x Q8_K
// ------------------------------------------------------------------------------------------------
// Work unit = (row, super-block) on 4 lanes: lane s = lane % 4 takes elements 64s .. 64s+63 of the
// super-block.  A block covers RB <= 16 * NP rows (16 units per wave per pass); RB is chosen so
// that there is about one block per CU, since every block quantizes all of x.  The nsb super-blocks of
// a row are dealt to the block's nw waves, wave w taking super-blocks w, w + nw, ... (SBW of
// them), so a wave quantizes x (MR token rows) only on its own super-blocks and into its own LDS
// records: no barrier separates the quantizer from the dot products.  Every weight load of a lane
// is issued before its quantizer runs.  A unit's integer sums are reduced over its 4 lanes (two DPP
// steps) and its fp32 term goes to LDS; after the block's one barrier, one thread per (token row,
// row) adds the terms over super-blocks in order, the oracle's sequence (bit-identical to it).
constexpr int KQ_REC = 256 + 64 + 16;   // one (token row, super-block) record: q[256] | bs[16] | d

// LDS bytes of a K-quant block: the waves' x records and the terms [MR][RB][nsb] (+ a spare).
__host__ __device__ constexpr size_t kq_lds(int MR, int RB, int nw, int sbw, int nsb)
{
    return (size_t)nw * sbw * MR * KQ_REC + ((size_t)MR * RB * nsb + 1) * 4;
}

// x of super-block sb (< nsb, else a load past the end: zeros) for token rows 0..MR-1 into the
// wave's records rec[MR].
template <int MR>
X100_DEV void kq_load_x(rsrc_t xr, int K, int sb, int nsb, float4 (&v)[MR])
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < MR; m++)
        v[m] = buf_load_f4(xr, sb < nsb ? (uint32_t)(m * K + sb * 256 + 4 * lane) * 4u : 0xfffffff0u);
}
template <int MR>
X100_DEV void kq_quant_x(const float4 (&v)[MR], uint8_t *rec)
{
#pragma unroll
    for (int m = 0; m < MR; m++)
        q8_K_wave(v[m], (int8_t *)(rec + m * KQ_REC), (int *)(rec + m * KQ_REC + 256), (float *)(rec + m * KQ_REC + 320));
}

// Sequential combine over super-blocks (same order and operations as the oracle).
template <int MR>
X100_DEV void kq_combine(int M, int N, int nsb, int RB, int row0, const float *tv, float *y)
{
    for (int t = threadIdx.x; t < MR * RB; t += blockDim.x) {
        const int m = t / RB, r = t - m * RB;
        if (m < M && row0 + r < N) {
            float acc = 0.0f;
            for (int sb = 0; sb < nsb; sb++) acc = acc + tv[(m * RB + r) * nsb + sb];
            y[(size_t)m * N + row0 + r] = acc;
        }
    }
}

// Q4_K: lane s holds qs bytes [32s, 32s+32) (low nibbles: sub-block 2s, high nibbles: sub-block
// 2s+1, get_scale_min_k4 of repack.cpp:222-233) and the 16-byte header (d, dmin, scales).
template <int MR, int NP, int SBW>
__global__ __launch_bounds__(512) void k_q4_K(int M, int N, int K, int RB, const uint8_t *__restrict__ W,
                                              const float *__restrict__ x, float *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nsb = K / 256, nw = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = wave_id(), s = lane & 3, ur = lane >> 2;
    const int row0 = blockIdx.x * RB;
    uint8_t *xw = smem + (size_t)w * SBW * MR * KQ_REC;
    float *tv = (float *)(smem + (size_t)nw * SBW * MR * KQ_REC);

    const rsrc_t xr = buf_rsrc(x, (uint32_t)(M * K) * 4u);
    float4 xv[MR];
    kq_load_x<MR>(xr, K, w, nsb, xv);

    // Unconditional loads (row and super-block clamped into the matrix; results discarded).
    v4i hdr[SBW][NP], q0[SBW][NP], q1[SBW][NP];
#pragma unroll
    for (int i = 0; i < SBW; i++)
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int sb = min(w + nw * i, nsb - 1), row = min(row0 + min(16 * p + ur, RB - 1), N - 1);
            const uint8_t *blk = W + ((size_t)row * nsb + sb) * 144;
            hdr[i][p] = *(const v4i *)blk;
            q0[i][p] = __builtin_nontemporal_load((const v4i *)(blk + 16 + 32 * s));
            q1[i][p] = __builtin_nontemporal_load((const v4i *)(blk + 32 + 32 * s));
        }
    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the quantizer
    kq_quant_x<MR>(xv, xw);
#pragma unroll
    for (int i = 1; i < SBW; i++) {
        kq_load_x<MR>(xr, K, w + nw * i, nsb, xv);
        kq_quant_x<MR>(xv, xw + i * MR * KQ_REC);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the wave's own LDS records
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
    for (int i = 0; i < SBW; i++) {
        const int sb = w + nw * i;
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int rl = 16 * p + ur;
            const bool valid = sb < nsb && rl < RB && row0 + rl < N;   // uniform over the unit's 4 lanes
            const uint32_t h0 = (uint32_t)hdr[i][p][0];
            const float d = h2f((uint16_t)(h0 & 0xffff)), dmin = h2f((uint16_t)(h0 >> 16));
            int sc0, m0, sc1, m1;
            scale_min_k4(2 * s, (uint32_t)hdr[i][p][1], (uint32_t)hdr[i][p][2], (uint32_t)hdr[i][p][3], sc0, m0);
            scale_min_k4(2 * s + 1, (uint32_t)hdr[i][p][1], (uint32_t)hdr[i][p][2], (uint32_t)hdr[i][p][3], sc1, m1);
            int lo[8], hi[8];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                lo[t] = q0[i][p][t] & 0x0F0F0F0F;
                hi[t] = (q0[i][p][t] >> 4) & 0x0F0F0F0F;
                lo[4 + t] = q1[i][p][t] & 0x0F0F0F0F;
                hi[4 + t] = (q1[i][p][t] >> 4) & 0x0F0F0F0F;
            }
#pragma unroll
            for (int m = 0; m < MR; m++) {
                // Branch-free: rows m >= M compute on zero records and are never combined; the 4
                // lanes of a unit store the same value; invalid units write the spare slot.
                const uint8_t *rec = xw + (i * MR + m) * KQ_REC;
                const v4i xa0 = *(const v4i *)(rec + 64 * s), xa1 = *(const v4i *)(rec + 64 * s + 16);
                const v4i xc0 = *(const v4i *)(rec + 64 * s + 32), xc1 = *(const v4i *)(rec + 64 * s + 48);
                const v4i bs = *(const v4i *)(rec + 256 + 16 * s);
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    d0 = dot4(lo[t], xa0[t], d0);
                    d0 = dot4(lo[4 + t], xa1[t], d0);
                    d1 = dot4(hi[t], xc0[t], d1);
                    d1 = dot4(hi[4 + t], xc1[t], d1);
                }
                const int isc = sum4_i(sc0 * d0 + sc1 * d1);
                const int imn = sum4_i(m0 * (bs[0] + bs[1]) + m1 * (bs[2] + bs[3]));
                const float dx = *(const float *)(rec + 320);
                const float dd = dx * d, dm = dx * dmin;
                tv[valid ? (m * RB + rl) * nsb + sb : MR * RB * nsb] = dd * (float)isc - dm * (float)imn;
            }
        }
    }
    __syncthreads();
    kq_combine<MR>(M, N, nsb, RB, row0, tv, y);
}

// Q3_K: lane s (hh = s / 2, lh = s % 2) loads qs bytes [32hh + 16lh, +16) and hmask bytes
// [16lh, +16) and decodes the 64 elements 128hh + 32j + 16lh + (0..15), j = 0..3 (shift 2j, hmask
// bit 4hh + j, scale index 8hh + 2j + lh), as dequantize_q3_K_block does (qwen_moe_q3k.c:565-575).
template <int MR, int NP, int SBW>
__global__ __launch_bounds__(512) void k_q3_K(int M, int N, int K, int RB, const uint8_t *__restrict__ hq,
                                              const uint8_t *__restrict__ scl,
                                              const uint16_t *__restrict__ wdd,
                                              const float *__restrict__ x, float *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nsb = K / 256, nw = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = wave_id(), s = lane & 3, ur = lane >> 2, hh = s >> 1, lh = s & 1;
    const int row0 = blockIdx.x * RB;
    uint8_t *xw = smem + (size_t)w * SBW * MR * KQ_REC;
    float *tv = (float *)(smem + (size_t)nw * SBW * MR * KQ_REC);

    const rsrc_t xr = buf_rsrc(x, (uint32_t)(M * K) * 4u);
    float4 xv[MR];
    kq_load_x<MR>(xr, K, w, nsb, xv);

    v4i qv[SBW][NP], hv[SBW][NP];
    uint32_t s0[SBW][NP], s1[SBW][NP], s2[SBW][NP], dv[SBW][NP];
#pragma unroll
    for (int i = 0; i < SBW; i++)
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int sb = min(w + nw * i, nsb - 1), row = min(row0 + min(16 * p + ur, RB - 1), N - 1);
            const size_t rec = (size_t)row * nsb + sb;
            qv[i][p] = __builtin_nontemporal_load((const v4i *)(hq + rec * 96 + 32 + 32 * hh + 16 * lh));
            hv[i][p] = *(const v4i *)(hq + rec * 96 + 16 * lh);
            const uint32_t *sp = (const uint32_t *)(scl + rec * 12);
            s0[i][p] = sp[0];
            s1[i][p] = sp[1];
            s2[i][p] = sp[2];
            dv[i][p] = wdd[rec];
        }
    __builtin_amdgcn_sched_barrier(0);
    kq_quant_x<MR>(xv, xw);
#pragma unroll
    for (int i = 1; i < SBW; i++) {
        kq_load_x<MR>(xr, K, w + nw * i, nsb, xv);
        kq_quant_x<MR>(xv, xw + i * MR * KQ_REC);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
    for (int i = 0; i < SBW; i++) {
        const int sb = w + nw * i;
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int rl = 16 * p + ur;
            const bool valid = sb < nsb && rl < RB && row0 + rl < N;
            int scv[4];
            int v[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                // 6-bit scale of sub-block is = 8hh + 2j + lh: low nibble of byte 2j + lh (hh = 0)
                // or its high nibble (hh = 1); high 2 bits from byte 8 + is % 4 at bit 2 (is / 4).
                const int k = 2 * j + lh, is = 8 * hh + k;
                const uint32_t low4 = (sbyte(s0[i][p], s1[i][p], s2[i][p], k) >> (4 * hh)) & 0xf;
                const uint32_t high2 = (sbyte(s0[i][p], s1[i][p], s2[i][p], 8 + (is & 3)) >> (2 * (is >> 2))) & 3;
                scv[j] = (int)(low4 | (high2 << 4)) - 32;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint32_t lo2 = ((uint32_t)qv[i][p][t] >> (2 * j)) & 0x03030303u;
                    const uint32_t hb = ((uint32_t)hv[i][p][t] >> (4 * hh + j)) & 0x01010101u;
                    v[j][t] = (int)(lo2 | (hb << 2));   // 3-bit value q + 4, q in [-4, 3]
                }
            }
            const float dw = h2f((uint16_t)dv[i][p]);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                // Branch-free, as in k_q4_K.
                const uint8_t *rec = xw + (i * MR + m) * KQ_REC;
                const int *bs = (const int *)(rec + 256) + 8 * hh + lh;
                int isc = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const v4i xq = *(const v4i *)(rec + 128 * hh + 32 * j + 16 * lh);
                    int dsum = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) dsum = dot4(v[j][t], xq[t], dsum);
                    dsum -= 4 * bs[2 * j];
                    isc += scv[j] * dsum;
                }
                isc = sum4_i(isc);
                const float dx = *(const float *)(rec + 320);
                tv[valid ? (m * RB + rl) * nsb + sb : MR * RB * nsb] = (dx * dw) * (float)isc;
            }
        }
    }
    __syncthreads();
    kq_combine<MR>(M, N, nsb, RB, row0, tv, y);
}

// ------------------------------------------------------------------------------------------------
// Q8_0 x int8 activation: the int8 path of Q8_0 / Q5_K / Q6_K weights
// ------------------------------------------------------------------------------------------------
// The weight was requantized to Q8_0 at load (k_requant_q8_0): d[N*nb] fp16 and qs[N*nb][32].
// x is quantized per 32 with an fp32 scale (pack_A_i8) and every 32-block contributes
// acc = fma(dw * scale, isum, acc), as run_i8_m1 does (qwen_moe_q3k.c:428-510).
//
// A row is owned by LPR = 16, 32 or 64 lanes (a wave holds 64/LPR row slots): lane j of a slot
// takes the 32-blocks j, j+LPR, ... (BPL per row), and the slot's sum is an in-row DPP prefix
// sum (plus row broadcasts for LPR > 16) that ends in the slot's last lane.  A row group is NT/64
// waves x RPW x 64/LPR rows.  Each block quantizes x once into LDS and then walks the row groups
// blockIdx.x, +gridDim.x, ...: the loads of the next group are issued before the current group's
// dot products, so a group's weights are always in flight while the previous one is reduced.
// Weight loads go through buffer resources: a row past N or a block past nb reads 0 without
// touching memory.  A row's arithmetic depends only on LPR and BPL (chosen from K), so a batch
// of M rows gives each row exactly what a one-row call gives.
template <int RPW, int BPL>
struct I8Group {
    v4i q[RPW][BPL][2];
    uint32_t d[RPW][BPL];
};

template <int LPR, int RPW, int NT>
X100_DEV int i8_row(int g, int w, int r, int lane)
{
    constexpr int SL = 64 / LPR;
    return g * ((NT / 64) * RPW * SL) + (w * RPW + r) * SL + lane / LPR;
}

template <int LPR, int RPW, int BPL, int NT>
X100_DEV void i8_load_group(I8Group<RPW, BPL> &t, int g, int N, int nb, rsrc_t qr, rsrc_t dr, uint32_t end)
{
    const int lane = threadIdx.x & 63, w = wave_id();
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            const int row = i8_row<LPR, RPW, NT>(g, w, r, lane), b = (lane % LPR) + LPR * c;
            const uint32_t blk = (row < N && b < nb) ? (uint32_t)row * (uint32_t)nb + (uint32_t)b : end;
            t.q[r][c][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(blk * 32u), 0, 0));
            t.q[r][c][1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(blk * 32u + 16u), 0, 0));
            t.d[r][c] = __builtin_amdgcn_raw_buffer_load_b16(dr, (int)(blk * 2u), 0, 0);
        }
}

// Sum over the LPR lanes of each row slot into the slot's last lane (inclusive prefix sum within
// rows of 16, then row broadcasts 15 and 31, the steps of wave_sum_uf).
template <int LPR>
X100_DEV float slot_sum(float v)
{
    v += dpp_f<0x111>(0.0f, v);
    v += dpp_f<0x112>(0.0f, v);
    v += dpp_f<0x114>(0.0f, v);
    v += dpp_f<0x118>(0.0f, v);
    if constexpr (LPR >= 32) v += dpp_f<0x142, 0xa>(0.0f, v);
    if constexpr (LPR >= 64) v += dpp_f<0x143, 0xc>(0.0f, v);
    return v;
}

template <int MR, int LPR, int RPW, int BPL, int XPT, int NT>
__global__ __launch_bounds__(NT) void k_q8_0(int M, int N, int K, int ngroups, const uint16_t *__restrict__ wd,
                                              const int8_t *__restrict__ wq, const float *__restrict__ x,
                                              float *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = K / 32;
    const int nb1 = MR * nb + 1;                 // + the quantizer's spare block
    int8_t *xlo = (int8_t *)smem;
    int8_t *xhi = xlo + nb1 * 16;
    float *xd = (float *)(xhi + nb1 * 16);
    int *xs = (int *)(xd + nb1);

    const int lane = threadIdx.x & 63, w = wave_id(), j = lane % LPR;
    const uint32_t nblk = (uint32_t)N * (uint32_t)nb;   // < 2^27 (checked by the launcher)
    const rsrc_t qr = buf_rsrc(wq, nblk * 32u);
    const rsrc_t dr = buf_rsrc(wd, nblk * 2u);

    const int total4 = M * K / 4;
    const rsrc_t xr = buf_rsrc(x, (uint32_t)total4 * 16u);
    float4 xv[XPT];
    x_load<XPT, NT>(xr, 0, xv);

    int g = blockIdx.x;
    I8Group<RPW, BPL> cur;
    i8_load_group<LPR, RPW, BPL, NT>(cur, g, N, nb, qr, dr, nblk);

    __builtin_amdgcn_sched_barrier(0);   // keep the first group's loads ahead of the quantizer
    q8_0_from_regs<XPT, NT, false>(xv, 0, total4, K, xlo, xhi, xd, xs);
    for (int c0 = NT * XPT; c0 < total4; c0 += NT * XPT) {
        x_load<XPT, NT>(xr, c0, xv);
        q8_0_from_regs<XPT, NT, false>(xv, c0, total4, K, xlo, xhi, xd, xs);
    }
    __syncthreads();

    for (; g < ngroups; g += gridDim.x) {
        I8Group<RPW, BPL> nxt;
        i8_load_group<LPR, RPW, BPL, NT>(nxt, g + (int)gridDim.x, N, nb, qr, dr, nblk);

        float acc[RPW][MR];
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int m = 0; m < MR; m++) acc[r][m] = 0.0f;
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            // A lane past the last block holds zero weights and a zero scale (its loads were out of
            // range), so fma(0, 0, acc) leaves its sum as it is: no branch, the LDS reads of all
            // blocks can be issued together.  Rows m >= M compute on unused LDS and are not stored.
            const int b = min(j + LPR * c, nb - 1);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const v4i xl = *(const v4i *)(xlo + (m * nb + b) * 16);
                const v4i xh = *(const v4i *)(xhi + (m * nb + b) * 16);
                const float sx = xd[m * nb + b];
#pragma unroll
                for (int r = 0; r < RPW; r++) {
                    int s = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        s = dot4(cur.q[r][c][0][t], xl[t], s);
                        s = dot4(cur.q[r][c][1][t], xh[t], s);
                    }
                    const float v1 = h2f((uint16_t)cur.d[r][c]) * sx;
                    acc[r][m] = __builtin_fmaf(v1, (float)s, acc[r][m]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int row = i8_row<LPR, RPW, NT>(g, w, r, lane);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                if (m < M) {
                    const float v = slot_sum<LPR>(acc[r][m]);
                    if (j == LPR - 1 && row < N) y[(size_t)m * N + row] = v;
                }
            }
        }
        cur = nxt;
    }
}

// ------------------------------------------------------------------------------------------------
// Weight packing (GGUF-native blocks -> device layout)
// ------------------------------------------------------------------------------------------------
__global__ void k_pack_q4_0(size_t nblk, const uint8_t *__restrict__ src, uint16_t *__restrict__ d,
                            uint8_t *__restrict__ qs)
{
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const uint8_t *s = src + b * 18;
    d[b] = (uint16_t)(s[0] | (s[1] << 8));
    uint8_t *o = qs + b * 16;
#pragma unroll
    for (int j = 0; j < 16; j++) o[j] = s[2 + j];
}

__global__ void k_pack_q3_K(size_t nblk, const uint8_t *__restrict__ src, uint8_t *__restrict__ hq,
                            uint8_t *__restrict__ scl, uint16_t *__restrict__ d)
{
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const uint8_t *s = src + b * 110;
    for (int j = 0; j < 96; j++) hq[b * 96 + j] = s[j];
    for (int j = 0; j < 12; j++) scl[b * 12 + j] = s[96 + j];
    d[b] = (uint16_t)(s[108] | (s[109] << 8));
}

// Load-time requantization to Q8_0 (lin_new_i8, qwen_moe_q3k.c:872-886): thread g dequantizes
// the 32-element group g from its GGUF block in fp32 with the operation order of
// gguf_dequant_into (qwen_moe_q3k.c:1129-1158; Q6_K qwen_moe.c:168-177) and re-encodes it with
// quantize_q8_0_native's rounding (amax floor 1e-6, d = amax/127, q = rint(w * (1/d)), d stored
// as fp16 rounded to nearest even).
template <int QT>
__global__ void k_requant_q8_0(size_t ngrp, const uint8_t *__restrict__ src, uint16_t *__restrict__ dq,
                               int8_t *__restrict__ qs)
{
    const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngrp) return;
    float v[32];
    if constexpr (QT == X100_Q8_0) {
        const uint8_t *b = src + g * 34;
        const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = (float)(int8_t)b[2 + j] * d;
    } else if constexpr (QT == X100_Q6_K) {
        // group gi of the super-block: half h = gi/4, quarter gg = gi%4 of the half.  Element l
        // takes the low (gg < 2) or high nibble of ql[64h + 32(gg%2) + l], bits 2gg, 2gg+1 of
        // qh[32h + l] and the int8 scale 8h + 2gg + l/16.
        const size_t sb = g >> 3;
        const int gi = (int)(g & 7), h = gi >> 2, gg = gi & 3;
        const uint8_t *b = src + sb * 210;
        const uint8_t *ql = b + 64 * h + 32 * (gg & 1), *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192) + 8 * h + 2 * gg;
        const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
        const int nsh = 4 * (gg >> 1), hsh = 2 * gg;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int q = (((ql[l] >> nsh) & 15) | (((qh[l] >> hsh) & 3) << 4)) - 32;
            v[l] = d * (float)sc[l >> 4] * (float)q;
        }
    } else {
        static_assert(QT == X100_Q5_K, "requant source type");
        // group gi = 2c + hi: low (hi = 0) or high nibbles of qs[32c + l], fifth bit = bit gi of
        // qh[l], (scale, min) pair gi.
        const size_t sb = g >> 3;
        const int gi = (int)(g & 7), c = gi >> 1, hi = gi & 1;
        const uint8_t *b = src + sb * 176;
        const float d = h2f((uint16_t)(b[0] | (b[1] << 8))), dmin = h2f((uint16_t)(b[2] | (b[3] << 8)));
        uint32_t s3[3];
#pragma unroll
        for (int i = 0; i < 3; i++)
            s3[i] = (uint32_t)b[4 + 4 * i] | ((uint32_t)b[5 + 4 * i] << 8) | ((uint32_t)b[6 + 4 * i] << 16) |
                    ((uint32_t)b[7 + 4 * i] << 24);
        int sc, m;
        scale_min_k4(gi, s3[0], s3[1], s3[2], sc, m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t *ql = b + 48 + 32 * c, *qh = b + 16;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int q = ((ql[l] >> (4 * hi)) & 15) + (((qh[l] >> gi) & 1) << 4);
            v[l] = d1 * (float)q - m1;
        }
    }
    float amax = 1e-6f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    dq[g] = f2h_trunc(d);   // quantize_q8_0_native's f32_to_f16 (qwen_moe_hp.c:71-79)
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t wv = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) wv |= (uint32_t)(clamp_i8((int)rintf(v[4 * j + i] * inv)) & 0xff) << (8 * i);
        pk[j] = wv;
    }
    uint4 *o = (uint4 *)(qs + g * 32);
    o[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    o[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
}

constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

// ------------------------------------------------------------------------------------------------
// Host-side layout helpers and launchers
// ------------------------------------------------------------------------------------------------
size_t x100_q_packed_bytes(int qtype, int N, int K)
{
    switch (qtype) {
    case X100_Q4_0: {
        const size_t nblk = (size_t)N * (K / 32);
        return align256(nblk * 2) + nblk * 16;
    }
    case X100_Q4_K: return (size_t)N * (K / 256) * 144;
    case X100_Q8_0: case X100_Q5_K: case X100_Q6_K: {
        const size_t ngrp = (size_t)N * (K / 32);
        return align256(ngrp * 2) + ngrp * 32;
    }
    case X100_Q3_K: {
        const size_t nblk = (size_t)N * (K / 256);
        return nblk * 96 + nblk * 12 + nblk * 2;
    }
    }
    return 0;
}

hipError_t x100_q_pack_launch(int qtype, int N, int K, const void *src, void *dst, hipStream_t s)
{
    switch (qtype) {
    case X100_Q4_0: {
        const size_t nblk = (size_t)N * (K / 32);
        uint16_t *d = (uint16_t *)dst;
        uint8_t *qs = (uint8_t *)dst + align256(nblk * 2);
        hipLaunchKernelGGL(k_pack_q4_0, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, nblk,
                           (const uint8_t *)src, d, qs);
        return hipGetLastError();
    }
    case X100_Q4_K:
        return hipMemcpyAsync(dst, src, (size_t)N * (K / 256) * 144, hipMemcpyDeviceToDevice, s);
    case X100_Q8_0: case X100_Q5_K: case X100_Q6_K: {
        const size_t ngrp = (size_t)N * (K / 32);
        uint16_t *d = (uint16_t *)dst;
        int8_t *qs = (int8_t *)dst + align256(ngrp * 2);
        const dim3 grid((unsigned)((ngrp + 255) / 256)), blk(256);
        const uint8_t *sp = (const uint8_t *)src;
        if (qtype == X100_Q8_0) hipLaunchKernelGGL(k_requant_q8_0<X100_Q8_0>, grid, blk, 0, s, ngrp, sp, d, qs);
        else if (qtype == X100_Q5_K) hipLaunchKernelGGL(k_requant_q8_0<X100_Q5_K>, grid, blk, 0, s, ngrp, sp, d, qs);
        else hipLaunchKernelGGL(k_requant_q8_0<X100_Q6_K>, grid, blk, 0, s, ngrp, sp, d, qs);
        return hipGetLastError();
    }
    case X100_Q3_K: {
        const size_t nblk = (size_t)N * (K / 256);
        uint8_t *hq = (uint8_t *)dst;
        uint8_t *scl = hq + nblk * 96;
        uint16_t *d = (uint16_t *)(scl + nblk * 12);
        hipLaunchKernelGGL(k_pack_q3_K, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, nblk,
                           (const uint8_t *)src, hq, scl, d);
        return hipGetLastError();
    }
    }
    return hipErrorInvalidValue;
}

namespace {


// Q4_0 block shape: one token row takes 4 waves of 4 rows each; several token rows take 16 waves
// of one row each (the same 16 rows per block, with the activation quantizer and the per-row dot
// products spread over four times as many waves) where the lane's blocks fit the 128 VGPRs of a
// 1024-thread block (BPL * MR <= 8).  BPL = 32-element blocks per lane per row.
inline int q40_bpl(int nb) { return nb <= 64 ? 1 : nb <= 128 ? 2 : nb <= 256 ? 4 : 8; }
constexpr bool q40_wide(int mr, int bpl) { return mr > 1 && bpl * mr <= 8; }

template <int MR, int BPL, int XPT>
void launch_q4_0_b(int M, int N, int K, const uint16_t *wd, const uint8_t *wq, size_t lds, const float *x,
                   float *y, hipStream_t s)
{
    constexpr int NT = q40_wide(MR, BPL) ? 1024 : 256, RPW = q40_wide(MR, BPL) ? 1 : 4;
    const int rows = (NT / 64) * RPW;
    const dim3 grid((N + rows - 1) / rows);
    hipLaunchKernelGGL((k_q4_0<MR, RPW, BPL, XPT, NT>), grid, dim3(NT), lds, s, M, N, K, wd, wq, x, y);
}

template <int MR, int XPT>
hipError_t launch_q4_0_x(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    const int nb = K / 32;
    const size_t nblk = (size_t)N * nb;
    const uint16_t *wd = (const uint16_t *)w;
    const uint8_t *wq = (const uint8_t *)w + align256(nblk * 2);
    const size_t lds = ((size_t)MR * nb + 1) * 40;
    switch (q40_bpl(nb)) {
    case 1: launch_q4_0_b<MR, 1, XPT>(M, N, K, wd, wq, lds, x, y, s); break;
    case 2: launch_q4_0_b<MR, 2, XPT>(M, N, K, wd, wq, lds, x, y, s); break;
    case 4: launch_q4_0_b<MR, 4, XPT>(M, N, K, wd, wq, lds, x, y, s); break;
    default: launch_q4_0_b<MR, 8, XPT>(M, N, K, wd, wq, lds, x, y, s); break;
    }
    return hipGetLastError();
}

template <int MR>
hipError_t launch_q4_0(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    // activation float4 per thread per pass, for the block's thread count
    const int nt = q40_wide(MR, q40_bpl(K / 32)) ? 1024 : 256;
    const int need = (M * K + 4 * nt - 1) / (4 * nt);
    if (need <= 2) return launch_q4_0_x<MR, 2>(M, N, K, w, x, y, s);
    if (need <= 4) return launch_q4_0_x<MR, 4>(M, N, K, w, x, y, s);
    if (need <= 8) return launch_q4_0_x<MR, 8>(M, N, K, w, x, y, s);
    return launch_q4_0_x<MR, 16>(M, N, K, w, x, y, s);
}

// Blocks of kernel k that are resident on the whole device at once with lds bytes of dynamic LDS
// (the runtime's occupancy for the kernel times the CU count): the grid of a persistent launch.
// Cached per kernel for the last (device, lds) pair of the calling thread.
template <typename Kern>
int resident_blocks(Kern k, int nt, size_t lds)
{
    static thread_local int c_dev = -1, c_blocks = 0;
    static thread_local size_t c_lds = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (dev != c_dev || lds != c_lds) {
        int occ = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, nt, lds) != hipSuccess || occ < 1) occ = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        c_dev = dev;
        c_lds = lds;
        c_blocks = occ * cus;
    }
    return c_blocks;
}

// int8 path: 256 threads.  Lanes per row LPR and blocks per lane BPL from nb = K/32 (a slot covers
// the row with at most 4 blocks per lane up to K = 8192); RPW row slots per wave so that a
// group's loads (RPW * BPL blocks of 34 B per lane, twice for the prefetch) stay within about 64
// VGPRs.  The grid is the number of blocks resident on the device at once, or one per row group
// if there are fewer groups.
template <int MR, int LPR, int BPL, int XPT>
hipError_t launch_q8_0_b(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    constexpr int NT = 256, RPW = BPL >= 4 ? 1 : 4 / BPL;
    const int nb = K / 32;
    const size_t ngrp = (size_t)N * nb;
    const uint16_t *wd = (const uint16_t *)w;
    const int8_t *wq = (const int8_t *)w + align256(ngrp * 2);
    const size_t lds = ((size_t)MR * nb + 1) * 40;
    const int rows = (NT / 64) * RPW * (64 / LPR);
    const int ngroups = (N + rows - 1) / rows;
    const int res = resident_blocks(k_q8_0<MR, LPR, RPW, BPL, XPT, NT>, NT, lds);
    const int grid = ngroups < res ? ngroups : res;
    hipLaunchKernelGGL((k_q8_0<MR, LPR, RPW, BPL, XPT, NT>), dim3(grid), dim3(NT), lds, s, M, N, K, ngroups, wd,
                       wq, x, y);
    return hipGetLastError();
}

template <int MR, int LPR, int BPL>
hipError_t launch_q8_0_x(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    const int need = (M * K + 4 * 256 - 1) / (4 * 256);
    if (need <= 2) return launch_q8_0_b<MR, LPR, BPL, 2>(M, N, K, w, x, y, s);
    if (need <= 4) return launch_q8_0_b<MR, LPR, BPL, 4>(M, N, K, w, x, y, s);
    if (need <= 8) return launch_q8_0_b<MR, LPR, BPL, 8>(M, N, K, w, x, y, s);
    return launch_q8_0_b<MR, LPR, BPL, 16>(M, N, K, w, x, y, s);
}

template <int MR>
hipError_t launch_q8_0(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    const int nb = K / 32;
    if (nb <= 16) return launch_q8_0_x<MR, 16, 1>(M, N, K, w, x, y, s);
    if (nb <= 32) return launch_q8_0_x<MR, 16, 2>(M, N, K, w, x, y, s);
    if (nb <= 64) return launch_q8_0_x<MR, 16, 4>(M, N, K, w, x, y, s);
    if (nb <= 128) return launch_q8_0_x<MR, 32, 4>(M, N, K, w, x, y, s);
    if (nb <= 256) return launch_q8_0_x<MR, 64, 4>(M, N, K, w, x, y, s);
    return launch_q8_0_x<MR, 64, 8>(M, N, K, w, x, y, s);
}

// K-quant launch plan: nw = min(nsb, 8) waves, SBW super-blocks per wave (a power of two, at most
// 8, so K <= 16384), RB = ceil(N / 256) rows per block (about one block per CU) but at least 16
// and at most 32 (two passes).  False when the block's LDS would exceed 160 KiB.
struct KqPlan {
    int nw, sbw, rb, np;
    size_t lds;
};
inline bool kq_plan(int MR, int N, int K, KqPlan &pl)
{
    const int nsb = K / 256;
    if (nsb < 1) return false;
    pl.nw = nsb < 8 ? nsb : 8;
    const int need = (nsb + pl.nw - 1) / pl.nw;
    pl.sbw = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
    if (need > 8) return false;
    pl.rb = min(32, max(16, (N + 255) / 256));
    pl.np = pl.sbw <= 4 ? (pl.rb + 15) / 16 : 1;   // eight super-blocks per wave: one pass
    if (pl.np == 1) pl.rb = 16;
    pl.lds = kq_lds(MR, pl.rb, pl.nw, pl.sbw, nsb);
    return pl.lds <= 160 * 1024;
}

template <int MR, bool Q3, int SBW, int NP>
hipError_t launch_kq_s(const KqPlan &pl, int M, int N, int K, const void *w, const float *x, float *y,
                       hipStream_t s)
{
    const dim3 grid((N + pl.rb - 1) / pl.rb), blk(64 * pl.nw);
    if constexpr (Q3) {
        const size_t nblk = (size_t)N * (K / 256);
        const uint8_t *hq = (const uint8_t *)w;
        const uint8_t *scl = hq + nblk * 96;
        const uint16_t *dd = (const uint16_t *)(scl + nblk * 12);
        hipLaunchKernelGGL((k_q3_K<MR, NP, SBW>), grid, blk, pl.lds, s, M, N, K, pl.rb, hq, scl, dd, x, y);
    } else {
        hipLaunchKernelGGL((k_q4_K<MR, NP, SBW>), grid, blk, pl.lds, s, M, N, K, pl.rb, (const uint8_t *)w, x, y);
    }
    return hipGetLastError();
}

template <int MR, bool Q3>
hipError_t launch_kq(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    KqPlan pl;
    if (!kq_plan(MR, N, K, pl)) return hipErrorInvalidValue;
    if (pl.np == 2) {
        switch (pl.sbw) {
        case 1: return launch_kq_s<MR, Q3, 1, 2>(pl, M, N, K, w, x, y, s);
        case 2: return launch_kq_s<MR, Q3, 2, 2>(pl, M, N, K, w, x, y, s);
        default: return launch_kq_s<MR, Q3, 4, 2>(pl, M, N, K, w, x, y, s);
        }
    }
    switch (pl.sbw) {
    case 1: return launch_kq_s<MR, Q3, 1, 1>(pl, M, N, K, w, x, y, s);
    case 2: return launch_kq_s<MR, Q3, 2, 1>(pl, M, N, K, w, x, y, s);
    case 4: return launch_kq_s<MR, Q3, 4, 1>(pl, M, N, K, w, x, y, s);
    default: return launch_kq_s<MR, Q3, 8, 1>(pl, M, N, K, w, x, y, s);
    }
}

}  // namespace

bool x100_qgemv_supported(int qtype, int M, int N, int K)
{
    if (M < 1 || M > 8 || N < 0 || K <= 0) return false;
    const size_t mr = M <= 1 ? 1 : (M <= 4 ? 4 : 8);
    if (qtype == X100_Q4_0)
        return K % 32 == 0 && K / 32 <= 512 && (mr * (K / 32) + 1) * 40 <= 160 * 1024;
    if (qtype == X100_Q8_0 || qtype == X100_Q5_K || qtype == X100_Q6_K)
        return K % (qtype == X100_Q8_0 ? 32 : 256) == 0 && K / 32 <= 512 && (mr * (K / 32) + 1) * 40 <= 160 * 1024 &&
               (size_t)N * (K / 32) < ((size_t)1 << 27);   // 32-bit buffer offsets
    if (qtype == X100_Q4_K || qtype == X100_Q3_K) {
        KqPlan pl;
        return K % 256 == 0 && kq_plan((int)mr, N, K, pl);
    }
    return false;
}

hipError_t x100_qgemv_launch(int qtype, int M, int N, int K, const void *w, const float *x, float *y,
                             hipStream_t s)
{
    if (!x100_qgemv_supported(qtype, M, N, K)) return hipErrorInvalidValue;
    if (qtype == X100_Q4_0) {
        if (M == 1) return launch_q4_0<1>(M, N, K, w, x, y, s);
        if (M <= 4) return launch_q4_0<4>(M, N, K, w, x, y, s);
        return launch_q4_0<8>(M, N, K, w, x, y, s);
    }
    if (qtype == X100_Q8_0 || qtype == X100_Q5_K || qtype == X100_Q6_K) {
        if (M == 1) return launch_q8_0<1>(M, N, K, w, x, y, s);
        if (M <= 4) return launch_q8_0<4>(M, N, K, w, x, y, s);
        return launch_q8_0<8>(M, N, K, w, x, y, s);
    }
    if (qtype == X100_Q4_K) {
        if (M == 1) return launch_kq<1, false>(M, N, K, w, x, y, s);
        if (M <= 4) return launch_kq<4, false>(M, N, K, w, x, y, s);
        return launch_kq<8, false>(M, N, K, w, x, y, s);
    }
    if (qtype == X100_Q3_K) {
        if (M == 1) return launch_kq<1, true>(M, N, K, w, x, y, s);
        if (M <= 4) return launch_kq<4, true>(M, N, K, w, x, y, s);
        return launch_kq<8, true>(M, N, K, w, x, y, s);
    }
    return hipErrorInvalidValue;
}
