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
//   Q4_0  split into d[N*K/32] (fp16) and qs[N*K/32][16], so nibble rows are 16-byte aligned.
//   Q4_K, Q3_K  super-block-major planes (see the K-quant section): 148 / 114 bytes per 256
//         elements (the GGUF blocks' 144 / 110 with the 6-bit scales unpacked to bytes).
//   Q8_0, Q5_K, Q6_K  requantized to Q8_0 (the reference loader's lin_new_i8) and split into
//         d[N*K/32] (fp16) and qs[N*K/32][32].
// Q4_0 keeps the GGUF blocks' byte count (plus alignment padding between the arrays); the int8
// path stores 34 bytes per 32 elements.
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
// (BPL per row).  All RPW*BPL nibble loads (16 B) and scale loads are issued first.  FULL: K is
// exactly 2048 * BPL, so every lane has all BPL blocks of a row and the LDS layout is known at
// compile time (no clamped block indices, no range selects, immediate LDS offsets).
template <int MR, int RPW, int BPL, int XPT, int NT, bool FULL>
__global__ __launch_bounds__(NT) void k_q4_0(int M, int N, int K, const uint16_t *__restrict__ wd,
                                              const uint8_t *__restrict__ wq,
                                              const float *__restrict__ x, float *__restrict__ y)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nb = FULL ? 64 * BPL : K / 32;
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
    // Several token rows: every wave's x loads go out before any wave's weight loads (an s_barrier,
    // no wait), so x, on which the quantizer and the barrier below wait, is not queued behind
    // the weights (M = 4: 6.02 -> 5.48 us; one row: no gain).
    if constexpr (MR > 1) __builtin_amdgcn_s_barrier();

    // Unconditional loads (indices clamped into the matrix; out-of-range results are discarded),
    // so every load of the lane is in flight before the first one is waited for.
    v4i q[RPW][BPL];
    uint32_t dwb[RPW][BPL];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            const int row = min(rowb + r, N - 1), b = FULL ? lane + 64 * c : min(lane + 64 * c, nb - 1);
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

    // Every row's lane partials first, then the row reductions, so that the rows' independent DPP
    // chains interleave (each row's order is unchanged).
    float acc[RPW][MR];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
#pragma unroll
        for (int m = 0; m < MR; m++) acc[r][m] = 0.0f;
#pragma unroll
        for (int c = 0; c < BPL; c++) {
            // Branch-free (the scheduler interleaves the unrolled blocks): a lane past the last
            // block reads block nb-1 and adds 0.  Rows m >= M compute on unused LDS and are not
            // stored.
            const bool inb = FULL || lane + 64 * c < nb;
            const int b = FULL ? lane + 64 * c : min(lane + 64 * c, nb - 1);
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
                int s = xs[m * nb + b];   // -8 * sum(x): the nibble offset, (q-8).x = q.x - 8*sum(x)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    s = dot4(lo[t], xl[t], s);
                    s = dot4(hi[t], xh[t], s);
                }
                const float term = (float)s * (dwf * xd[m * nb + b]);
                acc[r][m] += inb ? term : 0.0f;
            }
        }
    }
    float v[RPW * MR];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int m = 0; m < MR; m++) v[r * MR + m] = acc[r][m];
    wave_sum_uf_n(v);   // rows m >= M reduce unused values and are not stored
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int m = 0; m < MR; m++)
            if (m < M && lane == 0 && rowb + r < N) y[(size_t)m * N + rowb + r] = v[r * MR + m];
}

// ------------------------------------------------------------------------------------------------
// K-quants (Q4_K, Q3_K) x Q8_K
// ------------------------------------------------------------------------------------------------
// Device layout (made once by x100q_pack): one section per super-block column sb (all N rows),
// each section a set of planes in which the rows are contiguous, so that the lanes of a wave
// holding consecutive rows of one super-block read one contiguous run per load:
//   Q4_K section (148 bytes per row): 4 qs planes [N][2][16] (plane c, half h = qs bytes
//        64h + 16c .. +16 of the GGUF block), the scales [N][2][8] (half h: the 6-bit sc of
//        sub-blocks 4h .. 4h+3, then their 6-bit m, from get_scale_min_k4, repack.cpp:222-233),
//        d | dmin [N] (the block's first 4 bytes).
//   Q3_K section (114 bytes per row): 2 qs planes [N][2][16] (plane c, half h = qs bytes
//        32h + 16c .. +16), the high bits [N][2][16] (half h: bits 4h .. 4h+3 of the 32 hmask
//        bytes as nibbles, see k_pack_q3_K), the signed scales [N][2][8] (half h: scale - 32 of
//        sub-blocks 8h .. 8h+7, dequantize_q3_K_block, qwen_moe_q3k.c:557-577), d [N] (fp16).
// Every value is the GGUF block's own (no rounding): the layout only moves bits.
//
// Work unit = (row, super-block).  A block covers RB rows x all nsb super-blocks, RB about N / 256
// so that there is about one block per CU (every block quantizes all of x); its waves quantize the
// M x nsb Q8_K records of x into LDS between their weight loads and the first barrier.
//   k_q4_K4 / k_q3_K4 (several token rows, and one row when nsb is not 1, 2, 4 or 8): four lanes per
//     unit, units in super-block-major order (a wave's 16 units are consecutive rows of one or two
//     super-blocks); the quad reduces its integer sums with two DPP steps and stores the fp32
//     term; after the second barrier one thread per (token row, row) adds the terms over
//     super-blocks in order, the oracle's sequence (bit-identical to it).
//   k_kq_rm (one token row, nsb = 1, 2, 4 or 8): two lanes per unit (half h takes elements 128h ..
//     128h+127), units row-major, the sum over super-blocks inside the wave.

__host__ __device__ constexpr size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
__host__ __device__ constexpr size_t q4k_sec(int N) { return al256((size_t)148 * N); }
__host__ __device__ constexpr size_t q3k_sec(int N) { return al256((size_t)114 * N); }



// Arguments of the K-quant kernels (RB rows per block, nsb = K / 256 super-blocks per row).
struct KqArgs {
    int M, N, K, RB, nsb;
    uint32_t mrb, mnsb;   // udiv16 multipliers of RB and nsb
    const uint8_t *W;
    const float *x;
    float *y;
};

X100_DEV void q8k_load(rsrc_t xr, const KqArgs &a, int nq, int qb, float4 (&v)[4])
{
    q8k_load(xr, a.K, a.nsb, a.mnsb, nq, qb, v);
}

// The block's M x nsb records, passes of four: the wave with quantizer index w (a permutation of
// the wave ids) takes passes w, w + nw, w + 2nw, ...  The
// first two passes' loads are issued by q8k_first (before the weight loads), the rest are loaded
// and quantized one pass at a time by q8k_rest.
struct Q8kFirst {
    float4 v0[4], v1[4];
};
X100_DEV void q8k_first(rsrc_t xr, const KqArgs &a, int nq, int nw, Q8kFirst &f, int w)
{
    q8k_load(xr, a, nq, 4 * w, f.v0);
    if (4 * (w + nw) < nq) q8k_load(xr, a, nq, 4 * (w + nw), f.v1);
}
X100_DEV void q8k_rest(rsrc_t xr, const KqArgs &a, int nq, int nw, const Q8kFirst &f, uint8_t *recs, int w)
{
    q8k_quant(f.v0, nq, 4 * w, recs);
    if (4 * (w + nw) < nq) q8k_quant(f.v1, nq, 4 * (w + nw), recs);
    for (int qb = 4 * (w + 2 * nw); qb < nq; qb += 4 * nw) {
        float4 v[4];
        q8k_load(xr, a, nq, qb, v);
        q8k_quant(v, nq, qb, recs);
    }
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

// LDS bytes of a K-quant block: the MR*nsb records + a spare, then the terms [MR][RB][nsb] + a spare.
__host__ __device__ constexpr size_t kq_lds(int MR, int RB, int nsb)
{
    return (size_t)(MR * nsb + 1) * KREC + ((size_t)MR * RB * nsb + 1) * 4;
}

// The unit struct of the four-lanes-per-unit kernels (kq_unit4): u = sb * RB + r, clamped to the
// last unit; `valid` false for lanes past the block's units or rows past N.
struct KqUnit {
    int sb, r, row;
    bool valid;
};

// Several token rows, four lanes per unit: lane q = lane % 4 of unit u takes half h = q / 2 and,
// within it, the pair p = q % 2 of sub-blocks (Q4_K: planes 2p, 2p + 1 = sub-blocks 4h + 2p and
// 4h + 2p + 1; Q3_K: the even (p = 0) or odd (p = 1) sub-blocks 8h + 2j + p of the half).  Against
// two lanes per unit this halves every lane's chain of record reads and dot products per token
// row (the phase after the weights land), with 16 units per wave and up to 16 waves; the unit's
// integer sums are completed by two DPP steps across the quad (integer addition, so the same
// bits).  Q4_K 6144 x 2048, M = 4: 12 waves for 192 units.
X100_DEV KqUnit kq_unit4(const KqArgs &a)
{
    const int lane = threadIdx.x & 63, N = a.N, RB = a.RB, nu = RB * a.nsb;
    const int u0 = 16 * wave_id() + (lane >> 2), u = min(u0, nu - 1);
    KqUnit k;
    k.sb = (int)udiv16((uint32_t)u, (uint32_t)RB, a.mrb);
    k.r = u - k.sb * RB;
    const int row0 = blockIdx.x * RB;
    k.row = min(row0 + k.r, N - 1);
    k.valid = u0 < nu && row0 + k.r < N;
    return k;
}

// Sequential combine over NSB super-blocks (compile-time), each thread's terms read with 16-byte
// LDS loads; same order and operations as kq_combine.
template <int MR, int NSB>
X100_DEV void kq_combine_n(int M, int N, int RB, int row0, const float *tv, float *y)
{
    for (int t = threadIdx.x; t < MR * RB; t += blockDim.x) {
        const int m = t / RB, r = t - m * RB;
        if (m < M && row0 + r < N) {
            const float4 *tp = (const float4 *)(tv + (size_t)(m * RB + r) * NSB);
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NSB / 4; c++) {
                const float4 v = tp[c];
                acc = acc + v.x;
                acc = acc + v.y;
                acc = acc + v.z;
                acc = acc + v.w;
            }
            y[(size_t)m * N + row0 + r] = acc;
        }
    }
}
template <int MR>
X100_DEV void kq_combine_any(int M, int N, int nsb, int RB, int row0, const float *tv, float *y)
{
    if (nsb == 8)
        kq_combine_n<MR, 8>(M, N, RB, row0, tv, y);
    else if (nsb == 4)
        kq_combine_n<MR, 4>(M, N, RB, row0, tv, y);
    else
        kq_combine<MR>(M, N, nsb, RB, row0, tv, y);
}

template <int MR>
__global__ __launch_bounds__(1024) void k_q4_K4(const KqArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int M = a.M, N = a.N, RB = a.RB, nsb = a.nsb, nw = blockDim.x >> 6, nq = M * nsb;
    const uint8_t *__restrict__ W = a.W;
    const float *__restrict__ x = a.x;
    float *__restrict__ y = a.y;
    const int lane = threadIdx.x & 63, w = wave_id(), q = lane & 3, h = q >> 1, p = q & 1;
    uint8_t *recs = smem;
    float *tv = (float *)(smem + (size_t)(MR * nsb + 1) * KREC);
    const KqUnit ku = kq_unit4(a);

    const rsrc_t xr = buf_rsrc(x, (uint32_t)(M * a.K) * 4u);
    const bool wq = 4 * w < nq;   // the wave has records to quantize (wave-uniform)
    Q8kFirst xf;
    if (wq) q8k_first(xr, a, nq, nw, xf, w);
    // every wave's x loads before any wave's weight loads (s_barrier, no wait)
    __builtin_amdgcn_s_barrier();

    const uint8_t *sec = W + (size_t)ku.sb * q4k_sec(N);
    v4i qv[2];
#pragma unroll
    for (int c = 0; c < 2; c++)
        qv[c] = __builtin_nontemporal_load(
            (const v4i *)(sec + (size_t)(2 * p + c) * 32 * N + (size_t)ku.row * 32 + 16 * h));
    const uint2 smv = *(const uint2 *)(sec + (size_t)128 * N + (size_t)ku.row * 16 + 8 * h);
    const uint32_t ddv = *(const uint32_t *)(sec + (size_t)144 * N + (size_t)ku.row * 4);

    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the quantizer
    if (wq) q8k_rest(xr, a, nq, nw, xf, recs, w);
    __syncthreads();

    if (16 * w < RB * nsb) {   // waves past the block's units only quantized (wave-uniform)
        // sub-blocks j0 = 4h + 2p (low nibbles) and j0 + 1 (high nibbles)
        const int sc0 = (int)((smv.x >> (16 * p)) & 0xff), sc1 = (int)((smv.x >> (16 * p + 8)) & 0xff);
        const int mn0 = (int)((smv.y >> (16 * p)) & 0xff), mn1 = (int)((smv.y >> (16 * p + 8)) & 0xff);
        int lo[2][4], hi[2][4];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                lo[c][t] = qv[c][t] & 0x0F0F0F0F;
                hi[c][t] = (qv[c][t] >> 4) & 0x0F0F0F0F;
            }
        const float d = h2f((uint16_t)(ddv & 0xffff)), dmin = h2f((uint16_t)(ddv >> 16));
        const int spare = MR * RB * nsb;
#pragma unroll
        for (int m = 0; m < MR; m++) {
            // Branch-free: rows m >= M compute on unused LDS and are never combined.
            const uint8_t *rec = recs + (size_t)(m * nsb + ku.sb) * KREC;
            const v4i *xq = (const v4i *)(rec + 128 * h + 64 * p);
            const v4i x0 = xq[0], x1 = xq[1], x2 = xq[2], x3 = xq[3];
            const int2 s32 = *(const int2 *)(rec + KR_S32 + 16 * h + 8 * p);
            int da = 0, db = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                da = dot4(lo[0][t], x0[t], da);
                da = dot4(lo[1][t], x1[t], da);
                db = dot4(hi[0][t], x2[t], db);
                db = dot4(hi[1][t], x3[t], db);
            }
            int isc = sc0 * da + sc1 * db;
            int imn = mn0 * s32.x + mn1 * s32.y;
            isc += dpp_i<0xB1>(0, isc);   // + the pair's other lane (q ^ 1)
            imn += dpp_i<0xB1>(0, imn);
            isc += dpp_i<0x4E>(0, isc);   // + the other half (q ^ 2)
            imn += dpp_i<0x4E>(0, imn);
            tv[ku.valid ? (m * RB + ku.r) * nsb + ku.sb : spare] = q4k_term(d, dmin, *(const float *)(rec + KR_D), isc, imn);
        }
    }
    __syncthreads();
    kq_combine_any<MR>(M, N, nsb, RB, blockIdx.x * RB, tv, y);
}

template <int MR>
__global__ __launch_bounds__(1024) void k_q3_K4(const KqArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int M = a.M, N = a.N, RB = a.RB, nsb = a.nsb, nw = blockDim.x >> 6, nq = M * nsb;
    const uint8_t *__restrict__ W = a.W;
    const float *__restrict__ x = a.x;
    float *__restrict__ y = a.y;
    const int lane = threadIdx.x & 63, w = wave_id(), q = lane & 3, h = q >> 1, p = q & 1;
    uint8_t *recs = smem;
    float *tv = (float *)(smem + (size_t)(MR * nsb + 1) * KREC);
    const KqUnit ku = kq_unit4(a);

    const rsrc_t xr = buf_rsrc(x, (uint32_t)(M * a.K) * 4u);
    const bool wq = 4 * w < nq;   // the wave has records to quantize (wave-uniform)
    Q8kFirst xf;
    if (wq) q8k_first(xr, a, nq, nw, xf, w);
    __builtin_amdgcn_s_barrier();

    // plane p of the half: qs bytes 32h + 16p .. +16 (dword t: elements 128h + 32j + 16p + 4t ..
    // +3 at shift 2j, sub-block 8h + 2j + p); its high bits are the high-bit plane's dwords 2p, 2p+1
    const uint8_t *sec = W + (size_t)ku.sb * q3k_sec(N);
    const size_t ro = (size_t)ku.row * 32 + 16 * h;
    const v4i qp = __builtin_nontemporal_load((const v4i *)(sec + (size_t)32 * p * N + ro));
    const uint2 hm = *(const uint2 *)(sec + (size_t)64 * N + ro + 8 * p);
    const uint2 scv = *(const uint2 *)(sec + (size_t)96 * N + (size_t)ku.row * 16 + 8 * h);
    const uint16_t dw16 = *(const uint16_t *)(sec + (size_t)112 * N + (size_t)ku.row * 2);

    __builtin_amdgcn_sched_barrier(0);
    if (wq) q8k_rest(xr, a, nq, nw, xf, recs, w);
    __syncthreads();

    if (16 * w < RB * nsb) {   // waves past the block's units only quantized (wave-uniform)
        int sc[4];   // signed scales of sub-blocks 8h + 2j + p
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = (int)(int8_t)((((j < 2) ? scv.x : scv.y) >> (8 * (2 * (j & 1) + p))) & 0xff);
        int vq[4][4];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t hb = (((t >> 1) ? hm.y : hm.x) >> (4 * (t & 1) + j)) & 0x01010101u;
                vq[j][t] = (int)((((uint32_t)qp[t] >> (2 * j)) & 0x03030303u) | (hb << 2));
            }
        const float dw = h2f(dw16);
        const int spare = MR * RB * nsb;
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const uint8_t *rec = recs + (size_t)(m * nsb + ku.sb) * KREC;
            const v4i *xq = (const v4i *)(rec + 128 * h);
            const v4i sa = *(const v4i *)(rec + KR_S16 + 32 * h), sbv = *(const v4i *)(rec + KR_S16 + 32 * h + 16);
            const int s16[4] = {p ? sa[1] : sa[0], p ? sa[3] : sa[2], p ? sbv[1] : sbv[0], p ? sbv[3] : sbv[2]};
            int isc = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v4i xa = xq[2 * j + p];
                int dj = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) dj = dot4(vq[j][t], xa[t], dj);
                isc += sc[j] * (dj - 4 * s16[j]);
            }
            isc += dpp_i<0xB1>(0, isc);   // + the other parity (q ^ 1)
            isc += dpp_i<0x4E>(0, isc);   // + the other half (q ^ 2)
            const float dx = *(const float *)(rec + KR_D);
            tv[ku.valid ? (m * RB + ku.r) * nsb + ku.sb : spare] = (dx * dw) * (float)isc;
        }
    }
    __syncthreads();
    kq_combine_any<MR>(M, N, nsb, RB, blockIdx.x * RB, tv, y);
}

// Row-major kernel for one token row with nsb = 1, 2, 4 or 8 super-blocks per row, two lanes per
// unit (half h of the super-block, q4k_half_sums / the Q3_K half below): units u = row * nsb + sb,
// so that the 2 * nsb lanes of a row lie in one 16-lane DPP row.  Each unit's fp32 term
// (the same integers and operations as k_q4_K4 / k_q3_K4) is summed over the super-blocks in order by a chain
// of row_shr:2 steps inside the wave, starting from 0.0f + t0 as the oracle does, and the row's
// last unit writes y: no terms in LDS and no second barrier.  The weight loads of a wave cover
// 32 / nsb consecutive rows of every super-block section (whole 128-byte lines).
// ------------------------------------------------------------------------------------------------
// RMSNorm of one 2048-element row inside a 256-thread block, with the operations and order of
// k_rmsnorm<1024> (attn.hip): virtual thread T < 1024 sums h[T]^2 and h[T + 1024]^2 from 0, the 64
// virtual threads of a virtual wave reduce by wave_sum_bfly_f's butterfly, and the 16 wave sums are
// added in order; s = 1 / sqrtf(sum / 2048 + eps) and hn = h * s * w.  Thread t holds virtual
// threads 4t .. 4t+3 (its float4s at elements 4t and 1024 + 4t), so virtual lane 4 (t % 16) + j
// pairs with its butterfly partners l^32, l^16, l^8, l^4 in threads t^8, t^4, t^2, t^1 (component
// j) and with l^2, l^1 inside the thread.  Used where a row's norm is folded into its consumer.
// ------------------------------------------------------------------------------------------------
struct RmsRow {
    float4 a, b;
};
X100_DEV void rms_load(const float *__restrict__ h, RmsRow &r)
{
    r.a = *(const float4 *)(h + 4 * threadIdx.x);
    r.b = *(const float4 *)(h + 1024 + 4 * threadIdx.x);
}
// red: 16 floats of LDS; every thread of the block calls it (one barrier).
X100_DEV float rms_scale(const RmsRow &r, float eps, float *red)
{
    float v[4] = {0.0f + r.a.x * r.a.x, 0.0f + r.a.y * r.a.y, 0.0f + r.a.z * r.a.z, 0.0f + r.a.w * r.a.w};
    v[0] += r.b.x * r.b.x;
    v[1] += r.b.y * r.b.y;
    v[2] += r.b.z * r.b.z;
    v[3] += r.b.w * r.b.w;
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] += dpp_f<0x128>(0.0f, v[j]);   // t^8 (row_ror:8 within 16)
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] += dpp_f<0x124>(0.0f, v[j]);   // t^4 (values now depend on t % 8)
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] += dpp_f<0x4E>(0.0f, v[j]);    // t^2
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] += dpp_f<0xB1>(0.0f, v[j]);    // t^1
    const float u0 = v[0] + v[2], u1 = v[1] + v[3];                // virtual l^2
    const float tot16 = u0 + u1;                                   // virtual l^1
    if ((threadIdx.x & 15) == 0) red[threadIdx.x >> 4] = tot16;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) tot += red[k];
    return 1.0f / sqrtf(tot / 2048.0f + eps);
}
X100_DEV void rms_apply(float4 &v, float s, const float4 g)
{
    v.x = v.x * s * g.x;
    v.y = v.y * s * g.y;
    v.z = v.z * s * g.z;
    v.w = v.w * s * g.w;
}

// bx: the block's index within its matrix (blockIdx.x, or less in k_kq_rm2).
// NORM (one token row, K = 2048, every record in the first two passes): a.x is the raw row h, and
// the block applies RMSNorm with weights nrm (rms_scale, LDS at byte 4096) to the values it quantizes.
template <int MR, bool Q3, bool NORM = false>
X100_DEV void kq_rm_body(const KqArgs &a, int bx, const float *__restrict__ nrm = nullptr, float eps = 0.0f)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int M = a.M, N = a.N, K = a.K, RB = a.RB, nsb = a.nsb, nw = blockDim.x >> 6, nq = M * nsb;
    const uint8_t *__restrict__ W = a.W;
    const float *__restrict__ x = a.x;
    float *__restrict__ y = a.y;
    const int lane = threadIdx.x & 63, w = wave_id(), h = lane & 1;
    uint8_t *recs = smem;
    const int u0 = 32 * w + (lane >> 1), lgn = __builtin_ctz((unsigned)nsb);
    const int rib = u0 >> lgn, sb = u0 & (nsb - 1), row0 = bx * RB;
    const bool valid = rib < RB && row0 + rib < N;
    const int row = min(row0 + min(rib, RB - 1), N - 1);

    const rsrc_t xr = buf_rsrc(x, (uint32_t)(M * K) * 4u);
    // Quantizer index rotated by two: with 6 waves (one token row, 24 rows of 8 super-blocks) the
    // two quantizing waves are 2 and 3, alone on their SIMDs (waves map to SIMDs round-robin, so
    // 0-1 share theirs with dot waves 4-5): Q4_K 3.90 -> 3.84 us, Q3_K 3.89 -> 3.76 us.  Any
    // rotation is a permutation of the waves, so every record is still quantized once.
    const int qw = (w + nw - 2) % nw;
    const bool wq = 4 * qw < nq;   // the wave has records to quantize (wave-uniform)
    RmsRow rr;
    if constexpr (NORM) rms_load(x, rr);
    Q8kFirst xf;
    if (wq) q8k_first(xr, a, nq, nw, xf, qw);
    float4 g0[4], g1[4];   // the norm weights of the values in xf (elements as q8k_load takes them)
    if constexpr (NORM)
        if (wq) {
            const int e = 16 * (lane & 15);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int q0 = min(4 * qw + (lane >> 4), nq - 1), q1 = min(4 * (qw + nw) + (lane >> 4), nq - 1);
                g0[c] = *(const float4 *)(nrm + q0 * 256 + e + 4 * c);
                g1[c] = *(const float4 *)(nrm + q1 * 256 + e + 4 * c);
            }
        }

    v4i qv[4], hm = {};
    uint2 sv;
    uint32_t dv;
    if constexpr (!Q3) {
        const uint8_t *sec = W + (size_t)sb * q4k_sec(N);
#pragma unroll
        for (int c = 0; c < 4; c++)
            qv[c] = __builtin_nontemporal_load((const v4i *)(sec + (size_t)c * 32 * N + (size_t)row * 32 + 16 * h));
        sv = *(const uint2 *)(sec + (size_t)128 * N + (size_t)row * 16 + 8 * h);
        dv = *(const uint32_t *)(sec + (size_t)144 * N + (size_t)row * 4);
    } else {
        const uint8_t *sec = W + (size_t)sb * q3k_sec(N);
        const size_t ro = (size_t)row * 32 + 16 * h;
        qv[0] = __builtin_nontemporal_load((const v4i *)(sec + ro));
        qv[1] = __builtin_nontemporal_load((const v4i *)(sec + (size_t)32 * N + ro));
        hm = __builtin_nontemporal_load((const v4i *)(sec + (size_t)64 * N + ro));
        sv = *(const uint2 *)(sec + (size_t)96 * N + (size_t)row * 16 + 8 * h);
        dv = *(const uint16_t *)(sec + (size_t)112 * N + (size_t)row * 2);
    }

    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the quantizer
    if constexpr (NORM) {
        const float sc = rms_scale(rr, eps, (float *)(smem + 4096));
        if (wq) {
#pragma unroll
            for (int c = 0; c < 4; c++) rms_apply(xf.v0[c], sc, g0[c]);
            if (4 * (qw + nw) < nq)
#pragma unroll
                for (int c = 0; c < 4; c++) rms_apply(xf.v1[c], sc, g1[c]);
        }
    }
    if (wq) q8k_rest(xr, a, nq, nw, xf, recs, qw);
    __syncthreads();
    if (32 * w >= RB * nsb) return;   // waves past the block's units only quantized (wave-uniform)

    float term[MR];
    if constexpr (!Q3) {
        Q4kHalf u;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            u.sc[jj] = (int)((sv.x >> (8 * jj)) & 0xff);
            u.mn[jj] = (int)((sv.y >> (8 * jj)) & 0xff);
        }
        q4k_unpack(qv, u);
        const float d = h2f((uint16_t)(dv & 0xffff)), dmin = h2f((uint16_t)(dv >> 16));
#pragma unroll
        for (int m = 0; m < MR; m++) {
            // Rows m >= M compute on unused LDS and are never stored.
            const uint8_t *rec = recs + (size_t)(m * nsb + sb) * KREC;
            int isc, imn;
            q4k_half_sums(u, rec, h, isc, imn);
            term[m] = q4k_term(d, dmin, *(const float *)(rec + KR_D), isc, imn);
        }
    } else {
        int sc[8];
#pragma unroll
        for (int k = 0; k < 8; k++) sc[k] = (int)(int8_t)(((k < 4 ? sv.x : sv.y) >> (8 * (k & 3))) & 0xff);
        const uint32_t qd[8] = {(uint32_t)qv[0][0], (uint32_t)qv[0][1], (uint32_t)qv[0][2], (uint32_t)qv[0][3],
                                (uint32_t)qv[1][0], (uint32_t)qv[1][1], (uint32_t)qv[1][2], (uint32_t)qv[1][3]};
        int vq[4][8];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t hb = ((uint32_t)hm[t >> 1] >> (4 * (t & 1) + j)) & 0x01010101u;
                vq[j][t] = (int)(((qd[t] >> (2 * j)) & 0x03030303u) | (hb << 2));
            }
        const float dw = h2f((uint16_t)dv);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const uint8_t *rec = recs + (size_t)(m * nsb + sb) * KREC;
            const v4i *xq = (const v4i *)(rec + 128 * h);
            const v4i sa = *(const v4i *)(rec + KR_S16 + 32 * h), sbv = *(const v4i *)(rec + KR_S16 + 32 * h + 16);
            const int s16[8] = {sa[0], sa[1], sa[2], sa[3], sbv[0], sbv[1], sbv[2], sbv[3]};
            int isc = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v4i xa = xq[2 * j], xb = xq[2 * j + 1];
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    d0 = dot4(vq[j][t], xa[t], d0);
                    d1 = dot4(vq[j][4 + t], xb[t], d1);
                }
                isc += sc[2 * j] * (d0 - 4 * s16[2 * j]) + sc[2 * j + 1] * (d1 - 4 * s16[2 * j + 1]);
            }
            isc += dpp_i<0xB1>(0, isc);
            term[m] = (*(const float *)(rec + KR_D) * dw) * (float)isc;
        }
    }
    // y[m][row] = ((0 + t_0) + t_1) + ... + t_{nsb-1}: step k takes the running sum of unit k-1 (two
    // lanes down, row_shr:2) and adds t_k in the lanes of unit k.
#pragma unroll
    for (int m = 0; m < MR; m++) {
        float acc = sb == 0 ? 0.0f + term[m] : 0.0f;
#pragma unroll
        for (int k = 1; k < 8; k++)
            if (k < nsb) {
                const float prev = dpp_f<0x112>(acc, acc);
                acc = sb == k ? prev + term[m] : acc;
            }
        if (m < M && valid && h == 0 && sb == nsb - 1) y[(size_t)m * N + row] = acc;
    }
}

template <int MR, bool Q3>
__global__ __launch_bounds__(512) void k_kq_rm(const KqArgs a)
{
    kq_rm_body<MR, Q3>(a, blockIdx.x);
}

// Two one-row products of one weight type and the same x in one launch (the decode layer's q and
// v projections): blocks 0 .. nb0-1 compute a0, the rest a1, each block with its job's plan.
// Every row's result is that of k_kq_rm (the quantizer's records do not depend on which waves
// quantize them, and a row's sum is inside one wave).
template <bool Q3>
__global__ __launch_bounds__(512) void k_kq_rm2(const KqArgs a0, const KqArgs a1, int nb0)
{
    const bool first = (int)blockIdx.x < nb0;
    kq_rm_body<1, Q3>(first ? a0 : a1, first ? (int)blockIdx.x : (int)blockIdx.x - nb0);
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

// bx, gx: the block's index and the number of blocks among those that run this product (blockIdx.x
// and gridDim.x, or less in k_kq_rm2_q8); the block takes row groups bx, bx + gx, ...
// NORM (one token row, K = 2048, one pass of NT * XPT float4): x is the raw row h, and the block
// applies RMSNorm with weights nrm (rms_scale, LDS at byte 4096) to the values it quantizes.
template <int MR, int LPR, int RPW, int BPL, int XPT, int NT, bool NORM = false>
X100_DEV void q8_0_body(int M, int N, int K, int ngroups, const uint16_t *__restrict__ wd,
                        const int8_t *__restrict__ wq, const float *__restrict__ x, float *__restrict__ y, int bx,
                        int gx, const float *__restrict__ nrm = nullptr, float eps = 0.0f)
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
    RmsRow rr;
    if constexpr (NORM) rms_load(x, rr);
    float4 xv[XPT];
    x_load<XPT, NT>(xr, 0, xv);
    float4 gv[XPT];   // the norm weights of xv's elements
    if constexpr (NORM)
#pragma unroll
        for (int i = 0; i < XPT; i++) gv[i] = *(const float4 *)(nrm + 4 * (threadIdx.x + NT * i));

    int g = bx;
    I8Group<RPW, BPL> cur;
    i8_load_group<LPR, RPW, BPL, NT>(cur, g, N, nb, qr, dr, nblk);

    __builtin_amdgcn_sched_barrier(0);   // keep the first group's loads ahead of the quantizer
    if constexpr (NORM) {
        const float sc = rms_scale(rr, eps, (float *)(smem + 4096));
#pragma unroll
        for (int i = 0; i < XPT; i++) rms_apply(xv[i], sc, gv[i]);
    }
    q8_0_from_regs<XPT, NT, false, false>(xv, 0, total4, K, xlo, xhi, xd, xs);
    for (int c0 = NT * XPT; c0 < total4; c0 += NT * XPT) {
        x_load<XPT, NT>(xr, c0, xv);
        q8_0_from_regs<XPT, NT, false, false>(xv, c0, total4, K, xlo, xhi, xd, xs);
    }
    __syncthreads();

    for (; g < ngroups; g += gx) {
        I8Group<RPW, BPL> nxt;
        i8_load_group<LPR, RPW, BPL, NT>(nxt, g + gx, N, nb, qr, dr, nblk);

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

template <int MR, int LPR, int RPW, int BPL, int XPT, int NT>
__global__ __launch_bounds__(NT) void k_q8_0(int M, int N, int K, int ngroups, const uint16_t *__restrict__ wd,
                                              const int8_t *__restrict__ wq, const float *__restrict__ x,
                                              float *__restrict__ y)
{
    q8_0_body<MR, LPR, RPW, BPL, XPT, NT>(M, N, K, ngroups, wd, wq, x, y, blockIdx.x, gridDim.x);
}

// A decoder layer's q, v and k projections in one launch: blocks 0 .. nb0-1 compute a0 and
// nb0 .. nb01-1 a1 (one-row K-quant products, as k_kq_rm2), the rest the int8-path product of
// one token row with the plan of k_q8_0<1, 16, 1, 4, 2, 256> (33 to 64 blocks of 32 per row); each
// block does what it does in its own launch, so every result is that launch's.  256 threads.
// NORM: x (a0.x) is the layer's raw row h, and every block applies the attention RMSNorm (weights
// nrm, k_rmsnorm<1024>'s order) to the values it quantizes, in place of a norm launch before.
template <bool Q3, bool NORM>
__global__ __launch_bounds__(256) void k_kq_rm2_q8(const KqArgs a0, const KqArgs a1, int nb0, int nb01, int N2,
                                                   int ngroups2, const uint16_t *__restrict__ wd2,
                                                   const int8_t *__restrict__ wq2, float *__restrict__ y2,
                                                   const float *__restrict__ nrm, float eps)
{
    const int b = blockIdx.x;
    if (b < nb01)
        kq_rm_body<1, Q3, NORM>(b < nb0 ? a0 : a1, b < nb0 ? b : b - nb0, nrm, eps);
    else
        q8_0_body<1, 16, 1, 4, 2, 256, NORM>(1, N2, a0.K, ngroups2, wd2, wq2, a0.x, y2, b - nb01,
                                              (int)gridDim.x - nb01, nrm, eps);
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

// Q4_K GGUF blocks -> the planar layout of the K-quant GEMV kernels (one thread per (row, super-block) unit).
__global__ void k_pack_q4_K(int N, int nsb, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst)
{
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= (size_t)N * nsb) return;
    const int n = (int)(b / nsb), sb = (int)(b % nsb);
    const uint8_t *s = src + b * 144;
    uint8_t *sec = dst + (size_t)sb * q4k_sec(N);
    for (int c = 0; c < 4; c++)
        for (int h = 0; h < 2; h++)
            for (int k = 0; k < 16; k++) sec[(size_t)c * 32 * N + (size_t)n * 32 + 16 * h + k] = s[16 + 64 * h + 16 * c + k];
    // get_scale_min_k4 (repack.cpp:222-233) of sub-blocks j = 0..7: half j/4, sc at j%4, m at 4 + j%4
    const uint8_t *q = s + 4;
    uint8_t *sm = sec + (size_t)128 * N + (size_t)n * 16;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        if (j < 4) {
            sc = q[j] & 63;
            m = q[j + 4] & 63;
        } else {
            sc = (q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4);
            m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
        sm[8 * (j >> 2) + (j & 3)] = (uint8_t)sc;
        sm[8 * (j >> 2) + 4 + (j & 3)] = (uint8_t)m;
    }
    uint8_t *dd = sec + (size_t)144 * N + (size_t)n * 4;
    for (int k = 0; k < 4; k++) dd[k] = s[k];
}

// Q3_K GGUF blocks {hmask[32], qs[64], scales[12], d} -> the planar layout of the K-quant GEMVs.  The high
// bits of half h: nib(l) = bits 4h .. 4h+3 of hmask[l]; byte 4t' + b holds nib(8t' + b) in its
// low and nib(8t' + 4 + b) in its high nibble, so qs dword t of the half finds its four elements'
// bit j at bit 4(t % 2) + j of each byte of high-bit dword t / 2.
__global__ void k_pack_q3_K(int N, int nsb, const uint8_t *__restrict__ src, uint8_t *__restrict__ dst)
{
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= (size_t)N * nsb) return;
    const int n = (int)(b / nsb), sb = (int)(b % nsb);
    const uint8_t *s = src + b * 110;
    const uint8_t *hmask = s, *qs = s + 32, *scales = s + 96;
    uint8_t *sec = dst + (size_t)sb * q3k_sec(N);
    for (int c = 0; c < 2; c++)
        for (int h = 0; h < 2; h++)
            for (int k = 0; k < 16; k++) sec[(size_t)c * 32 * N + (size_t)n * 32 + 16 * h + k] = qs[32 * h + 16 * c + k];
    for (int h = 0; h < 2; h++) {
        uint8_t *hb = sec + (size_t)64 * N + (size_t)n * 32 + 16 * h;
        for (int t = 0; t < 4; t++)
            for (int k = 0; k < 4; k++) {
                const int lo = (hmask[8 * t + k] >> (4 * h)) & 15, hi = (hmask[8 * t + 4 + k] >> (4 * h)) & 15;
                hb[4 * t + k] = (uint8_t)(lo | (hi << 4));
            }
    }
    // the 6-bit scale of sub-block is (dequantize_q3_K_block, qwen_moe_q3k.c:557-577) minus 32
    int8_t *sc = (int8_t *)(sec + (size_t)96 * N + (size_t)n * 16);
    for (int is = 0; is < 16; is++) {
        const int low4 = (scales[is & 7] >> (4 * (is >> 3))) & 15;
        const int high2 = (scales[8 + (is & 3)] >> (2 * (is >> 2))) & 3;
        sc[is] = (int8_t)((low4 | (high2 << 4)) - 32);
    }
    uint8_t *d = sec + (size_t)112 * N + (size_t)n * 2;
    d[0] = s[108];
    d[1] = s[109];
}

// Load-time requantization to Q8_0 (lin_new_i8, qwen_moe_q3k.c:872-886): thread g dequantizes
// the 32-element group g from its GGUF block in fp32 with the operation order of
// gguf_dequant_into (qwen_moe_q3k.c:1129-1158; Q6_K qwen_moe.c:168-177) and re-encodes it with
// quantize_q8_0_native's rounding (amax floor 1e-6, d = amax/127, q = rint(w * (1/d)), d stored
// as fp16 by the reference's truncating f32_to_f16, qwen_moe_hp.c:71-79).
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
    case X100_Q4_K: return (size_t)(K / 256) * q4k_sec(N);
    case X100_Q8_0: case X100_Q5_K: case X100_Q6_K: {
        const size_t ngrp = (size_t)N * (K / 32);
        return align256(ngrp * 2) + ngrp * 32;
    }
    case X100_Q3_K: return (size_t)(K / 256) * q3k_sec(N);
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
    case X100_Q4_K: case X100_Q3_K: {
        const size_t nblk = (size_t)N * (K / 256);
        const dim3 grid((unsigned)((nblk + 255) / 256)), blk(256);
        if (qtype == X100_Q4_K)
            hipLaunchKernelGGL(k_pack_q4_K, grid, blk, 0, s, N, K / 256, (const uint8_t *)src, (uint8_t *)dst);
        else
            hipLaunchKernelGGL(k_pack_q3_K, grid, blk, 0, s, N, K / 256, (const uint8_t *)src, (uint8_t *)dst);
        return hipGetLastError();
    }
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
    if (K == 2048 * BPL)
        hipLaunchKernelGGL((k_q4_0<MR, RPW, BPL, XPT, NT, true>), grid, dim3(NT), lds, s, M, N, K, wd, wq, x, y);
    else
        hipLaunchKernelGGL((k_q4_0<MR, RPW, BPL, XPT, NT, false>), grid, dim3(NT), lds, s, M, N, K, wd, wq, x, y);
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

// K-quant launch plan: RB = ceil(N / 256) rows per block (about one block per CU), at most 256 / nsb
// (so at most 16 waves of 16 four-lane units); nw = the waves of the two-lane row-major kernel;
// false when the block's LDS would exceed 160 KiB.
struct KqPlan {
    int rb, nw;
    size_t lds;
};
inline bool kq_plan(int MR, int N, int K, KqPlan &pl)
{
    const int nsb = K / 256;
    if (nsb < 1 || nsb > 256) return false;
    pl.rb = min(max(1, (N + 255) / 256), 256 / nsb);
    // waves for the units, or more (at most 8) so that every wave quantizes at most one pass of
    // four x records; waves past the units only quantize
    pl.nw = min(8, max((2 * pl.rb * nsb + 63) / 64, (MR * nsb + 3) / 4));
    pl.lds = kq_lds(MR, pl.rb, nsb);
    return pl.lds <= 160 * 1024;
}

template <int MR, bool Q3>
hipError_t launch_kq(int M, int N, int K, const void *w, const float *x, float *y, hipStream_t s)
{
    KqPlan pl;
    if (!kq_plan(MR, N, K, pl)) return hipErrorInvalidValue;
    const dim3 grid((N + pl.rb - 1) / pl.rb), blk(64 * pl.nw);
    const KqArgs a{M, N, K, pl.rb, K / 256, udiv16_magic((uint32_t)pl.rb), udiv16_magic((uint32_t)(K / 256)),
                   (const uint8_t *)w, x, y};
    // One token row with nsb = 1, 2, 4 or 8 (a row's units within one DPP row): the row-major form
    // (Q4_K 6144 x 2048: 3.86 vs 3.93 us; with several rows its per-row add chains cost more than
    // the barrier and combine they replace: 6.09 vs 5.47 us at M = 4).
    const int nsb = K / 256;
    if (MR == 1 && (nsb == 1 || nsb == 2 || nsb == 4 || nsb == 8)) {
        hipLaunchKernelGGL((k_kq_rm<MR, Q3>), grid, blk, (size_t)(MR * nsb + 1) * KREC, s, a);
    } else {
        // four lanes per unit: waves for the units (16 per wave; rb * nsb <= 256), or more so that
        // every wave quantizes at most one pass of four records, at most 16
        const dim3 blk4(64 * min(16, max((4 * pl.rb * nsb + 63) / 64, (MR * nsb + 3) / 4)));
        if constexpr (Q3)
            hipLaunchKernelGGL(k_q3_K4<MR>, grid, blk4, pl.lds, s, a);
        else
            hipLaunchKernelGGL(k_q4_K4<MR>, grid, blk4, pl.lds, s, a);
    }
    return hipGetLastError();
}

// Plans of two matrices in one launch: both take the larger rows per block of the two.  kq_plan
// sizes a matrix for a launch of its own (about 256 blocks), and every block of a shared launch
// quantizes all of x, so the smaller matrix (the 512 rows of a v projection beside 4096 of q: 256
// blocks of 2 rows) would add as many blocks of that fixed work as the larger one for a tenth of
// its weights.
inline void kq_plan_shared(int K, KqPlan &p0, KqPlan &p1)
{
    const int nsb = K / 256, rb = max(p0.rb, p1.rb);
    for (KqPlan *p : {&p0, &p1}) {
        p->rb = rb;
        p->nw = min(8, max((2 * rb * nsb + 63) / 64, (nsb + 3) / 4));
        p->lds = kq_lds(1, rb, nsb);
    }
}

// y0 = W0 x and y1 = W1 x for one token row, both Q4_K or both Q3_K with K / 256 in {1, 2, 4, 8},
// in one launch of k_kq_rm2 (hipErrorNotSupported otherwise: the caller launches them one by one).
template <bool Q3>
hipError_t launch_kq2(int N0, const void *w0, float *y0, int N1, const void *w1, float *y1, int K, const float *x,
                      hipStream_t s)
{
    const int nsb = K / 256;
    KqPlan p0, p1;
    if (K % 256 || !(nsb == 1 || nsb == 2 || nsb == 4 || nsb == 8) || !kq_plan(1, N0, K, p0) || !kq_plan(1, N1, K, p1))
        return hipErrorNotSupported;
    kq_plan_shared(K, p0, p1);
    const KqArgs a0{1, N0, K, p0.rb, nsb, udiv16_magic((uint32_t)p0.rb), udiv16_magic((uint32_t)nsb),
                    (const uint8_t *)w0, x, y0};
    const KqArgs a1{1, N1, K, p1.rb, nsb, udiv16_magic((uint32_t)p1.rb), udiv16_magic((uint32_t)nsb),
                    (const uint8_t *)w1, x, y1};
    const int nb0 = (N0 + p0.rb - 1) / p0.rb, nb1 = (N1 + p1.rb - 1) / p1.rb;
    hipLaunchKernelGGL(k_kq_rm2<Q3>, dim3(nb0 + nb1), dim3(64 * max(p0.nw, p1.nw)), (size_t)(nsb + 1) * KREC, s, a0,
                       a1, nb0);
    return hipGetLastError();
}

// y0 = W0 x, y1 = W1 x (both Q4_K or both Q3_K) and y2 = W2 x (int8 path) for one token row in one
// launch of k_kq_rm2_q8, when K = 2048 (the K-quant row-major form with 8 super-blocks and the
// int8 plan that kernel instantiates) and both K-quant plans use 4 waves; hipErrorNotSupported
// otherwise (nothing launched).
template <bool Q3>
hipError_t launch_kq2_q8(int N0, const void *w0, float *y0, int N1, const void *w1, float *y1, int N2, const void *w2,
                         float *y2, int K, const float *x, const float *nrm, float eps, hipStream_t s)
{
    const int nsb = K / 256, nb = K / 32;
    KqPlan p0, p1;
    if (K != 2048 || N2 < 1 || (size_t)N2 * nb >= ((size_t)1 << 27) || !kq_plan(1, N0, K, p0) || !kq_plan(1, N1, K, p1))
        return hipErrorNotSupported;
    kq_plan_shared(K, p0, p1);
    if (max(p0.nw, p1.nw) != 4) return hipErrorNotSupported;
    const KqArgs a0{1, N0, K, p0.rb, nsb, udiv16_magic((uint32_t)p0.rb), udiv16_magic((uint32_t)nsb),
                    (const uint8_t *)w0, x, y0};
    const KqArgs a1{1, N1, K, p1.rb, nsb, udiv16_magic((uint32_t)p1.rb), udiv16_magic((uint32_t)nsb),
                    (const uint8_t *)w1, x, y1};
    const int nb0 = (N0 + p0.rb - 1) / p0.rb, nb1 = (N1 + p1.rb - 1) / p1.rb;
    // the int8 product as launch_q8_0_b lays it out: 16 rows per group (4 waves x 64 / 16 lanes),
    // one block per group (fewer groups than resident blocks)
    const size_t ngrp = (size_t)N2 * nb;
    const int ngroups = (N2 + 15) / 16;
    const size_t lds = max(max((size_t)(nsb + 1) * KREC, ((size_t)nb + 1) * 40), (size_t)4096 + 16 * 4);
    const uint16_t *wd = (const uint16_t *)w2;
    const int8_t *wq = (const int8_t *)w2 + align256(ngrp * 2);
    if (nrm)
        hipLaunchKernelGGL((k_kq_rm2_q8<Q3, true>), dim3(nb0 + nb1 + ngroups), dim3(256), lds, s, a0, a1, nb0,
                           nb0 + nb1, N2, ngroups, wd, wq, y2, nrm, eps);
    else
        hipLaunchKernelGGL((k_kq_rm2_q8<Q3, false>), dim3(nb0 + nb1 + ngroups), dim3(256), lds, s, a0, a1, nb0,
                           nb0 + nb1, N2, ngroups, wd, wq, y2, nrm, eps);
    return hipGetLastError();
}

// Exhaustive check of the activation quantizer's division-free arithmetic (x100_common.h) on the
// device: for every float u in [lo, hi] (bit patterns), cnt[0] counts rcp_rn_any(u) != 1.0f / u
// (rcp_rn_any is rcp_rn from 2^-126 up, so this covers both), cnt[1] div127_rn(u) != u / 127.0f
// and cnt[2] f16_trunc_pos(u) != the reference's fp16
// truncation (f2h_trunc then h2f).  The divisions here are IEEE (built with correctly rounded
// division).
__global__ __launch_bounds__(256) void k_check_quant_div(uint32_t lo, uint32_t hi, unsigned long long *cnt)
{
    unsigned long long c0 = 0, c1 = 0, c2 = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = (uint64_t)lo + blockIdx.x * blockDim.x + threadIdx.x; u <= hi; u += stride) {
        const float v = __uint_as_float((uint32_t)u);
        c0 += __float_as_uint(rcp_rn_any(v)) != __float_as_uint(1.0f / v);
        c1 += __float_as_uint(div127_rn(v)) != __float_as_uint(v / 127.0f);
        c2 += __float_as_uint(f16_trunc_pos(v)) != __float_as_uint(h2f(f2h_trunc(v)));
    }
    atomicAdd(&cnt[0], c0);
    atomicAdd(&cnt[1], c1);
    atomicAdd(&cnt[2], c2);
}

}  // namespace

hipError_t x100_qgemv2_launch(int qtype, int N0, const void *w0, float *y0, int N1, const void *w1, float *y1, int K,
                              const float *x, hipStream_t s)
{
    if (N0 < 1 || N1 < 1) return hipErrorNotSupported;
    if (qtype == X100_Q4_K) return launch_kq2<false>(N0, w0, y0, N1, w1, y1, K, x, s);
    if (qtype == X100_Q3_K) return launch_kq2<true>(N0, w0, y0, N1, w1, y1, K, x, s);
    return hipErrorNotSupported;
}

hipError_t x100_qgemv3_launch(int qtype, int N0, const void *w0, float *y0, int N1, const void *w1, float *y1,
                              int qtype2, int N2, const void *w2, float *y2, int K, const float *x, const float *nrm,
                              float eps, hipStream_t s)
{
    if (N0 < 1 || N1 < 1 || !(qtype2 == X100_Q8_0 || qtype2 == X100_Q5_K || qtype2 == X100_Q6_K))
        return hipErrorNotSupported;
    if (qtype == X100_Q4_K) return launch_kq2_q8<false>(N0, w0, y0, N1, w1, y1, N2, w2, y2, K, x, nrm, eps, s);
    if (qtype == X100_Q3_K) return launch_kq2_q8<true>(N0, w0, y0, N1, w1, y1, N2, w2, y2, K, x, nrm, eps, s);
    return hipErrorNotSupported;
}

hipError_t x100_check_quant_div_launch(uint32_t lo, uint32_t hi, unsigned long long *cnt, hipStream_t s)
{
    hipLaunchKernelGGL(k_check_quant_div, dim3(4096), dim3(256), 0, s, lo, hi, cnt);
    return hipGetLastError();
}

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
