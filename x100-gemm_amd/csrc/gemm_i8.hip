// int8 x int8 -> int32 GEMM for gfx950:  C[MxN] += A[MxK] . B[KxN], all row-major.
//
// Replaces the reference's gemm_ime_i8 (src/gemm_ime_i8.c:60-89) whose IME micro-kernel is a stub
// that falls back to the scalar gemm_ref_i8 (src/gemm_ref.c:17-26).  Integer arithmetic is exact,
// so every kernel here is bit-identical to gemm_ref_i8 for any K below 2^17 (|sum| < 2^31).
//
// Three kernels:
//   k_gemm_mfma    tiled MFMA kernel (v_mfma_i32_32x32x32_i8).  A tiles go to LDS row-major with
//                  an XOR swizzle on 16-byte chunks; B tiles are transposed in registers
//                  (v_perm_b32) into "k-quad" dwords (4 consecutive k of one column) so that both
//                  MFMA operands are k-contiguous.  Double-buffered LDS, C loaded into the
//                  accumulators (C += A.B), XCD-aware grouped tile order.
//   k_gemm_skinny  M <= 16 rows (speculative-verify shapes): HBM-bound on B.  Split-K over
//                  256-row chunks, B streamed once through LDS, dot4 on transposed k-quads,
//                  int32 atomics into C (exact and order independent).
//   k_gemm_generic any shape / alignment (byte loads); correctness fallback.
#include <type_traits>

#include "x100_common.h"
#include "x100_internal.h"

namespace {

constexpr int BK = 64;  // k bytes per pipeline stage

// Tile order: blocks are dealt to the 8 XCDs round-robin, so block b runs on XCD b%8.  Give each
// XCD a contiguous range of tile ids, and walk tile ids in groups of GROUP_M tile rows so the
// tiles of one XCD share A row panels and B column panels in its L2.
X100_DEV void tile_coords(int bid, int nblk, int tiles_m, int tiles_n, int &tm, int &tn)
{
    int t = bid;
    if ((nblk & 7) == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
    constexpr int GROUP_M = 4;
    int per_group = GROUP_M * tiles_n;
    int g = t / per_group;
    int first_m = g * GROUP_M;
    int gsize = min(tiles_m - first_m, GROUP_M);
    int r = t - g * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// A tile in LDS: BM rows x 64 bytes; 16-byte chunk c of row r stored at chunk c ^ ((r>>1)&3)
// so that 8 consecutive lanes reading one chunk column hit 8 distinct 16-byte bank groups.
X100_DEV int a_lds_off(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 3)) << 4); }

template <int FM, int FN, int WM, int WN, bool EDGE, bool ACC>
__global__ __launch_bounds__(WM *WN * 64) void k_gemm_mfma(int M, int N, int K,
                                                           const int8_t *__restrict__ A,
                                                           const int8_t *__restrict__ B,
                                                           int32_t *__restrict__ C, int tiles_m,
                                                           int tiles_n)
{
    constexpr int NT = WM * WN * 64;
    constexpr int BM = WM * FM * 32;
    constexpr int BN = WN * FN * 32;
    constexpr int A_IT = BM * 4 / NT;             // 16-byte A chunks per thread per stage
    constexpr int B_UNITS = BN;                   // (k-quad, 16 columns) units per stage
    constexpr int B_IT = (B_UNITS + NT - 1) / NT;
    static_assert(A_IT * NT == BM * 4, "A tile must split evenly over the threads");

    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * BK];
    __shared__ __attribute__((aligned(16))) uint32_t Bs[2][16 * BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lcol = lane & 31, lgrp = lane >> 5;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // EDGE = false is only launched when M % BM == 0, N % BN == 0 and K % BK == 0.
    const bool full_mn = !EDGE || ((m0 + BM <= M) && (n0 + BN <= N));

    // Accumulators start from C (ACC: C += A.B) or from zero (C = A.B, C never read).  32x32 MFMA
    // output layout: lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int gn = n0 + wn * FN * 32 + 32 * j + lcol;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int gm = m0 + wm * FM * 32 + 32 * i + 8 * (r >> 2) + 4 * lgrp + (r & 3);
                acc[i][j][r] = (ACC && (full_mn || (gm < M && gn < N))) ? C[(size_t)gm * N + gn] : 0;
            }
        }

    v4i ra[A_IT];
    v4i rb[B_IT][4];

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
        const bool full = !EDGE || (full_mn && (k0 + BK <= K));
#pragma unroll
        for (int p = 0; p < A_IT; p++) {
            const int ch = tid + p * NT, r = ch >> 2, c = ch & 3;
            const int gm = m0 + r, gk = k0 + 16 * c;
            if (full || (gm < M && gk < K))
                ra[p] = *(const v4i *)(A + (size_t)gm * K + gk);
            else
                ra[p] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int p = 0; p < B_IT; p++) {
            const int u = tid + p * NT;
            if (B_UNITS % NT == 0 || u < B_UNITS) {
                const int kq = u / (BN / 16), nc = u % (BN / 16);
                const int gn = n0 + 16 * nc;
#pragma unroll
                for (int rr = 0; rr < 4; rr++) {
                    const int gk = k0 + 4 * kq + rr;
                    if (full || (gk < K && gn < N))
                        rb[p][rr] = *(const v4i *)(B + (size_t)gk * N + gn);
                    else
                        rb[p][rr] = v4i{0, 0, 0, 0};
                }
            }
        }
    };

    auto lstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < A_IT; p++) {
            const int ch = tid + p * NT, r = ch >> 2, c = ch & 3;
            *(v4i *)(&As[buf][a_lds_off(r, c)]) = ra[p];
        }
#pragma unroll
        for (int p = 0; p < B_IT; p++) {
            const int u = tid + p * NT;
            if (B_UNITS % NT == 0 || u < B_UNITS) {
                const int kq = u / (BN / 16), nc = u % (BN / 16);
                uint32_t o[16];
#pragma unroll
                for (int cg = 0; cg < 4; cg++)
                    transpose4x4((uint32_t)rb[p][0][cg], (uint32_t)rb[p][1][cg],
                                 (uint32_t)rb[p][2][cg], (uint32_t)rb[p][3][cg], o[4 * cg + 0],
                                 o[4 * cg + 1], o[4 * cg + 2], o[4 * cg + 3]);
                v4u *dst = (v4u *)(&Bs[buf][kq * BN + 16 * nc]);
                dst[0] = v4u{o[0], o[1], o[2], o[3]};
                dst[1] = v4u{o[4], o[5], o[6], o[7]};
                dst[2] = v4u{o[8], o[9], o[10], o[11]};
                dst[3] = v4u{o[12], o[13], o[14], o[15]};
            }
        }
    };

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int r = wm * FM * 32 + 32 * i + lcol;
                af[i] = *(const v4i *)(&As[buf][a_lds_off(r, 2 * kk + lgrp)]);
            }
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = wn * FN * 32 + 32 * j + lcol;
                const int kq = 8 * kk + 4 * lgrp;
                const uint32_t *bp = &Bs[buf][kq * BN + n];
                bf[j] = v4i{(int)bp[0], (int)bp[BN], (int)bp[2 * BN], (int)bp[3 * BN]};
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int gn = n0 + wn * FN * 32 + 32 * j + lcol;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int gm = m0 + wm * FM * 32 + 32 * i + 8 * (r >> 2) + 4 * lgrp + (r & 3);
                if (full_mn || (gm < M && gn < N)) C[(size_t)gm * N + gn] = acc[i][j][r];
            }
        }
}

// ------------------------------------------------------------------------------------------------
// Large-tile kernel: 256x256 output tile per block, NW waves (2 x NW/2; 8 waves = two per SIMD,
// 128x64 each), K step 64.
//
// * Operands reach LDS by direct global->LDS DMA (global_load_lds_dwordx4: lane l's 16 bytes land
//   at M0 + 16*l), through a 4-stage ring refilled as soon as a stage is consumed; the loads are
//   issued from inline asm so the compiler does not drain them at every barrier, and each
//   iteration waits with an exact s_waitcnt vmcnt for the stage it is about to read.
// * A tile: 256 rows x 64 bytes, 16-byte chunk c of row r stored at chunk big_a_chunk(r, c);
//   fragments read with ds_read_b128 (k-contiguous rows, conflict-free).
// * B tile: 64 k-rows x 256 bytes, row-major as in memory, chunk c of k-row k stored at
//   big_b_chunk(k, c);
//   fragments read with ds_read_b64_tr_b8 (lane c of each 16-lane group receives column c of an
//   8x16 byte block), two reads give the 16 consecutive k of one column that MFMA wants.
// * MFMA operands are swapped (B fragment first) so the accumulator holds C^T: each lane owns
//   4 consecutive C columns per register quad, and C is read and written 16 bytes at a time.
// * C += A.B: the accumulators start at zero; the old C is prefetched a quarter of the tile at a
//   time (before the K loop, then at 1/4, 1/2, 3/4 of it) and added when the next quarter is
//   fetched, so C reads overlap the MFMA work.
// Requires M % 256 == 0, N % 256 == 0, K % 64 == 0, K >= 512, 16-byte aligned pointers.
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;


// LDS swizzles for a 64-bank (256 bytes per cycle) LDS: ds_read_b128 serves 16 lanes and
// ds_read_b64_tr_b8 32 lanes per cycle, so those lanes must hit distinct 16-byte granules of a
// 256-byte bank row.
//   A (64-byte rows): 16 consecutive rows, same chunk c -> granule 4*(r&3) + (c ^ ((r>>2)&3)).
//   B (256-byte k-rows): 8 consecutive k, chunks c and c+1 (c even) -> c ^ 2*(k&7) and its ^1.
X100_DEV int big_a_chunk(int r, int c) { return c ^ ((r >> 2) & 3); }
X100_DEV int big_b_chunk(int k, int c) { return c ^ (2 * (k & 7)); }
//   A of a two-stage superslot (128-byte rows, whole cache lines): 16 consecutive rows, same
//   chunk c -> granule 8*(r&1) + (c ^ ((r>>1)&7)).
X100_DEV int big_a2_chunk(int r, int c) { return c ^ ((r >> 1) & 7); }

// Global -> LDS DMA of 16 bytes per lane: a wave-uniform 64-bit base address plus a 32-bit per-lane
// byte offset.  The LDS destination (wave-uniform) is passed in M0 through the "{m0}" operand, so
// the compiler knows the register is written.
X100_DEV void dma16s(uint32_t voff, const void *sbase, uint32_t lds_base)
{
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

template <int N> X100_DEV void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Wait until at most n of this wave's vector-memory operations are outstanding.
X100_DEV void wait_vmcnt_le(int n)
{
    // Largest listed count <= n (waiting for more completions than needed is always safe).
    if (n >= 56) wait_vmcnt<56>();
    else if (n >= 48) wait_vmcnt<48>();
    else if (n >= 40) wait_vmcnt<40>();
    else if (n >= 32) wait_vmcnt<32>();
    else if (n >= 24) wait_vmcnt<24>();
    else if (n >= 16) wait_vmcnt<16>();
    else if (n >= 12) wait_vmcnt<12>();
    else if (n >= 8) wait_vmcnt<8>();
    else if (n >= 4) wait_vmcnt<4>();
    else wait_vmcnt<0>();
}

X100_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte global store of a finished C chunk with the system-scope policy bits (sc0 sc1): C is
// written once and not read back by the kernel, and this form measured 69.5 -> 68.5 us at
// 4096^3 (a plain store, the same bits on a buffer store and nt all measured slower).  The
// trailing s_nop 1 gives the two wait states that gfx950 requires between a store of more than
// 8 bytes and a VALU write to its data registers (the compiler's own hazard recognizer emits
// s_nop 1 for this pattern on gfx950); the compiler does not add them after inline asm.  The
// compiler does not count this store in vmcnt either, so no vector-memory load may follow it in
// the kernel.
X100_DEV void store_c16(int32_t *dst, v4i v)
{
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" ::"v"(dst), "v"(v) : "memory");
}

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (indices usable as constants).
template <int I, int N, class F> X100_DEV void static_for_impl(F &&f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_impl<I + 1, N>(f);
    }
}
template <int N, class F> X100_DEV void static_for(F &&f) { static_for_impl<0, N>(f); }

template <int NW, int SUPER, bool ACC>
__global__ __launch_bounds__(NW * 64) void k_gemm_big(int M, int N, int K, const int8_t *__restrict__ A,
                                                     const int8_t *__restrict__ B,
                                                     int32_t *__restrict__ C, int tiles_m, int tiles_n)
{
    // NW waves as 2 x NW/2; each wave owns 128 rows x FN*32 columns of the 256x256 tile.
    constexpr int NS = 4, STAGE = 32768, BOFF = 16384;
    constexpr int WN = NW / 2, FN = 8 / WN;   // column fragments per wave
    constexpr int OPS = 16 / NW;              // DMA ops per wave per operand per stage
    __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t csm[NW * 4096];   // C staging, 4 KiB per wave

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w / WN, wn = w % WN, lcol = lane & 31, lgrp = lane >> 5;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * 256, n0 = tn * 256;
    const int nk = K / 64;

    // DMA sources: A op p covers tile rows 16*(NW*p+w) .. +15 (lane -> row lane/4, chunk lane%4),
    // B op p covers k-rows 4*(NW*p+w) .. +3 (lane -> row lane/16, chunk lane%16); each lane fetches
    // the logical chunk whose swizzled position is its own.
    const int8_t *Ab = A + (size_t)m0 * K;
    const int8_t *Bb = B + n0;
    // With SUPER == 2 the A rows of both stages of a superstage are fetched together as 128-byte
    // rows (op p covers tile rows 8*(NW*p+w) .. +7: lane -> row lane/8, chunk lane%8), so every
    // A fetch is a whole cache line instead of two half lines fetched a stage apart.
    // Op p differs from op 0 by a whole number of swizzle periods of rows, so the per-lane offset
    // is the same for every op and the op's row shift goes into the scalar base address.
    constexpr int AOPS = SUPER == 2 ? 2 * OPS : OPS;
    constexpr int AROWS = SUPER == 2 ? 8 : 16;   // tile rows per A op
    uint32_t aoff, boff;
    if constexpr (SUPER == 2) {
        const int ra = 8 * w + (lane >> 3);
        aoff = (uint32_t)(ra * K + 16 * big_a2_chunk(ra, lane & 7));
    } else {
        const int ra = 16 * w + (lane >> 2);
        aoff = (uint32_t)(ra * K + 16 * big_a_chunk(ra, lane & 3));
    }
    {
        const int rb = 4 * w + (lane >> 4);
        boff = (uint32_t)(rb * N + 16 * big_b_chunk(rb, lane & 15));
    }
    const uint32_t sbase = lds_addr(smem);
    auto dma_a = [&](const int8_t *ak, int p, uint32_t lds) __attribute__((always_inline)) {
        dma16s(aoff, ak + (size_t)AROWS * NW * p * K, lds);
    };
    auto dma_b = [&](const int8_t *bk, int p, uint32_t lds) __attribute__((always_inline)) {
        dma16s(boff, bk + (size_t)4 * NW * p * N, lds);
    };
    // Stage kt (clamped to the last stage: the loop issues 4 stages ahead unconditionally, and a
    // stage past the end is never read) into ring slot kt % NS.
    auto issue = [&](int kt) __attribute__((always_inline)) {
        const uint32_t sb = sbase + (uint32_t)((kt & (NS - 1)) * STAGE);
        const int kc = min(kt, nk - 1);
        const int8_t *ak = Ab + (size_t)kc * 64;
        const int8_t *bk = Bb + (size_t)kc * 64 * N;
#pragma unroll
        for (int p = 0; p < OPS; p++)
            dma_a(ak, p, __builtin_amdgcn_readfirstlane(sb + (uint32_t)(16 * (NW * p + w) * 64)));
#pragma unroll
        for (int p = 0; p < OPS; p++)
            dma_b(bk, p, __builtin_amdgcn_readfirstlane(sb + BOFF + (uint32_t)(4 * (NW * p + w) * 256)));
    };
    // SUPER == 2: superstage u (stages 2u, 2u+1; clamped like issue) into superslot u % 2 =
    // [A 256 rows x 128 bytes | B of stage 2u | B of stage 2u+1].
    auto issue_super = [&](int u) __attribute__((always_inline)) {
        const uint32_t sb = sbase + (uint32_t)((u & 1) * 2 * STAGE);
        const int uc = min(u, nk / 2 - 1);
        const int8_t *ak = Ab + (size_t)uc * 128;
#pragma unroll
        for (int p = 0; p < AOPS; p++)
            dma_a(ak, p, __builtin_amdgcn_readfirstlane(sb + (uint32_t)(8 * (NW * p + w) * 128)));
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int8_t *bk = Bb + (size_t)(2 * uc + h) * 64 * N;
#pragma unroll
            for (int p = 0; p < OPS; p++)
                dma_b(bk, p, __builtin_amdgcn_readfirstlane(sb + STAGE + h * BOFF + (uint32_t)(4 * (NW * p + w) * 256)));
        }
    };

    // C prefetch by parts: part p = accumulator fragment (i, j) = (p / FN, p % FN) of the wave,
    // 32 C rows x 32 columns (128 bytes).  Each part reaches a
    // wave-private 4 KiB LDS area by global->LDS DMA: 4 ops, each 8 rows x 128 bytes (whole cache
    // lines), 16-byte chunk c of row r stored at chunk big_a2_chunk(r, c) so that the accumulator-
    // layout reads below (16 rows, same chunk) are conflict-free.  No VGPRs hold C in flight.
    constexpr int NPART = 4 * FN;
    uint32_t coff[2];   // op t: row 8t + lane/8; ops t and t+2 differ by 16 rows (one swizzle period)
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int r = 8 * t + (lane >> 3);
        coff[t] = (uint32_t)(4 * ((wm * 128 + r) * N + wn * FN * 32 + 4 * big_a2_chunk(r, lane & 7)));
    }
    const uint32_t cl = lds_addr(csm) + (uint32_t)(w * 4096);
    auto load_c = [&](int p) __attribute__((always_inline)) {
        const int i = p / FN, j = p % FN;
        const int32_t *cb = C + (size_t)(m0 + 32 * i) * N + n0 + 32 * j;
#pragma unroll
        for (int t = 0; t < 4; t++)
            dma16s(coff[t & 1], cb + (size_t)16 * (t >> 1) * N,
                   __builtin_amdgcn_readfirstlane(cl + (uint32_t)(1024 * t)));
    };

    v16i acc[4][FN];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // pend: vector-memory ops of this wave issued after part p's DMA (waited for exactly).
    auto add_c = [&](auto pc, int pend) __attribute__((always_inline)) {   // pc: compile-time part index
        constexpr int p = decltype(pc)::value;
        constexpr int i = p / FN, j = p % FN;
        wait_vmcnt_le(pend);
        v4i cv[4];
        const uint8_t *cw = csm + w * 4096 + lcol * 128;
#pragma unroll
        for (int q = 0; q < 4; q++) cv[q] = *(const v4i *)(cw + 16 * big_a2_chunk(lcol, 2 * q + lgrp));
        // The adds below are inline asm, for which the compiler inserts no hazard wait states:
        // keep every MFMA above this point and wait out the MFMA-result-to-VALU latency (a
        // 16-pass MFMA needs 18 wait states; 32 are given) before reading accumulators.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // Integer add written as asm: a plain += makes the register allocator move
                // all the accumulators between register files (and spill); this keeps them
                // where the MFMAs want them (ArchVGPRs with 8 waves, AGPRs with 4).
                int x = acc[i][j][4 * q + e];
                if constexpr (NW == 8) {
                    asm volatile("v_add_u32 %0, %0, %1" : "+v"(x) : "v"(cv[q][e]));
                } else {
                    int t;
                    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_add_u32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                                 : "+a"(x), "=&v"(t) : "v"(cv[q][e]));
                }
                acc[i][j][4 * q + e] = x;
            }
    };

    // B fragment addressing for ds_read_b64_tr_b8: 16-lane group G = lane/16 covers columns
    // 16*(G&1) .. +15 of the 32-column fragment and k-rows 16*(G>>1) + 8t + (lane%16)/2.
    const int q16 = lane & 15, r8 = q16 >> 1, h8 = q16 & 1, ch = (lane >> 4) & 1;
    auto read_frags = [&](int slot, int kk, v4i (&af)[4], v4i (&bf)[FN]) __attribute__((always_inline)) {
        const uint8_t *As = SUPER == 2 ? smem + (slot >> 1) * 2 * STAGE : smem + slot * STAGE;
        const uint8_t *Bs = SUPER == 2 ? As + STAGE + (slot & 1) * BOFF : As + BOFF;
        auto read_a = [&](int i) __attribute__((always_inline)) {
            const int r = wm * 128 + 32 * i + lcol;
            if constexpr (SUPER == 2)
                af[i] = *(const v4i *)(As + r * 128 + 16 * big_a2_chunk(r, 4 * (slot & 1) + 2 * kk + lgrp));
            else
                af[i] = *(const v4i *)(As + r * 64 + 16 * big_a_chunk(r, 2 * kk + lgrp));
        };
        // In the order of first use by mma (row fragment outer): A0, every B fragment, A1..A3.
        read_a(0);
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int c = 2 * FN * wn + 2 * j + ch;
            const int k0 = 32 * kk + 16 * lgrp + r8;
            const uint8_t *p0 = Bs + k0 * 256 + 16 * big_b_chunk(r8, c) + 8 * h8;
            const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(const lds_u8 *)p0);
            const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(const lds_u8 *)(p0 + 8 * 256));
            bf[j] = v4i{lo.x, lo.y, hi.x, hi.y};
        }
#pragma unroll
        for (int i = 1; i < 4; i++) read_a(i);
    };
    auto mma = [&](const v4i (&af)[4], const v4i (&bf)[FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
    };

    // Software pipeline.  Iteration kt: read k-half 1 of stage kt, MFMAs on k-half 0; wait for
    // stage kt+1 and barrier (all waves are then done reading stage kt, whose slot is refilled
    // with stage kt+4); read k-half 0 of stage kt+1; MFMAs on k-half 1.  LDS reads are always
    // one MFMA group ahead of their use.
    // The K loop runs in NPART segments; C part p is added at the end of segment p, when part
    // p+1 is prefetched (part 0 right after the prologue's DMAs).
    constexpr int DPS = 2 * OPS;      // DMA ops per wave per stage
    constexpr int CQ = ACC ? 4 : 0;   // C DMA ops per wave per part (none in the overwrite form)
    // Vector-memory operations of this wave issued after stage s+1's DMAs when iteration s waits
    // for them: stages s+2 and s+3 (always issued: the prologue issues 0..3, step t issues t+4),
    // C part 0 (issued after the prologue's 4 stages, so after stage s+1 when s+1 <= 3) and every
    // C part p >= 1 whose load (after step ev_p - 1) lies between stage s+1's issue (prologue,
    // or step s-3) and step s.
    auto pending_after = [&](int s) __attribute__((always_inline)) {
        int n = 2 * DPS;
        if (s + 1 <= 3) n += CQ;
        for (int p = 1; p < NPART; p++) {
            const int t = p * nk / NPART - 1;
            if ((s + 1 <= 3 || t >= s - 3) && t <= s - 1) n += CQ;
        }
        return n;
    };
    // Instruction order inside each half-step: the ds_reads of the next fragments alternate with
    // the MFMAs of the current ones, so LDS latency hides behind the matrix pipe even with one
    // wave per SIMD.
    constexpr int NRD = 4 + 2 * FN, NMF = 4 * FN;
    auto interleave = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < NRD; r++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        }
        if constexpr (NMF > NRD) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD, 0);
    };
    v4i a0[4], b0[FN], a1[4], b1[FN];
    auto step = [&](int kt) __attribute__((always_inline)) {   // kt < nk - 1
        read_frags(kt & (NS - 1), 1, a1, b1);
        mma(a0, b0);
        interleave();
        wait_vmcnt_le(pending_after(kt));
        lds_barrier();
        issue(kt + 4);
        read_frags((kt + 1) & (NS - 1), 0, a0, b0);
        mma(a1, b1);
        interleave();
    };
    auto last_step = [&]() __attribute__((always_inline)) {   // kt = nk - 1
        read_frags((nk - 1) & (NS - 1), 1, a1, b1);
        mma(a0, b0);
        mma(a1, b1);
    };
    // Two stages per barrier (SUPER == 2, K % 128 == 0): superstage u = stages 2u, 2u+1.  On
    // entry slots hold 2u, 2u+1 (complete) and 2u+2, 2u+3 (in flight); before the only barrier of
    // the superstage the wave waits for 2u+2 and 2u+3, and after it refills the slots of 2u and
    // 2u+1 with 2u+4 and 2u+5.  Outstanding operations allowed at that wait: C parts loaded after
    // stage 2u+3 was issued (at the previous superstage's barrier), i.e. part 0 for u = 0 and a
    // part p loaded at the end of superstage u-1.
    const int nsup = nk / 2;
    auto pending_super = [&](int u) __attribute__((always_inline)) {
        int n = u == 0 ? CQ : 0;
        for (int p = 1; p < NPART; p++)
            if (p * nsup / NPART - 1 == u - 1) n += CQ;
        return n;
    };
    // The last k-half of a superstep with superstage u's DMA ops (issue_super's, same order)
    // spread between its MFMAs: issued as one burst after the barrier, the 8 waves' DMA ops back up
    // the vector-memory queue and every wave stalls at issue while the matrix pipe runs dry.
    auto mma_dma = [&](const v4i (&af)[4], const v4i (&bf)[FN], int u) __attribute__((always_inline)) {
        const uint32_t sb = sbase + (uint32_t)((u & 1) * 2 * STAGE);
        const int uc = min(u, nk / 2 - 1);
        const int8_t *ak = Ab + (size_t)uc * 128;
        static_for<4 * FN>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value, i = c / FN, j = c % FN;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            static_for<(AOPS + 2 * OPS) / (4 * FN)>([&](auto dd) __attribute__((always_inline)) {
                constexpr int k = c * ((AOPS + 2 * OPS) / (4 * FN)) + decltype(dd)::value;
                if constexpr (k < AOPS) {
                    dma_a(ak, k, __builtin_amdgcn_readfirstlane(sb + (uint32_t)(8 * (NW * k + w) * 128)));
                } else {
                    constexpr int h = (k - AOPS) / OPS, q = (k - AOPS) % OPS;
                    dma_b(Bb + (size_t)(2 * uc + h) * 64 * N, q,
                          __builtin_amdgcn_readfirstlane(sb + STAGE + h * BOFF + (uint32_t)(4 * (NW * q + w) * 256)));
                }
            });
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    auto superstep = [&](int u) __attribute__((always_inline)) {   // u < nsup - 1
        const int s0 = (2 * u) & (NS - 1), s1 = (2 * u + 1) & (NS - 1);
        read_frags(s0, 1, a1, b1);
        mma(a0, b0);
        interleave();
        read_frags(s1, 0, a0, b0);
        mma(a1, b1);
        interleave();
        read_frags(s1, 1, a1, b1);
        mma(a0, b0);
        interleave();
        wait_vmcnt_le(pending_super(u));
        lds_barrier();
        read_frags((2 * u + 2) & (NS - 1), 0, a0, b0);
        mma_dma(a1, b1, u + 2);
    };
    auto last_super = [&]() __attribute__((always_inline)) {   // u = nsup - 1
        const int s0 = (nk - 2) & (NS - 1), s1 = (nk - 1) & (NS - 1);
        read_frags(s0, 1, a1, b1);
        mma(a0, b0);
        interleave();
        read_frags(s1, 0, a0, b0);
        mma(a1, b1);
        interleave();
        read_frags(s1, 1, a1, b1);
        mma(a0, b0);
        mma(a1, b1);
    };
    if constexpr (SUPER == 2) {
        issue_super(0);
        issue_super(1);
    } else {
        issue(0);
        issue(1);
        issue(2);
        issue(3);
    }
    if constexpr (ACC) load_c(0);
    if constexpr (SUPER == 2) {
        wait_vmcnt_le(2 * DPS + CQ);   // stages 0 and 1 complete
        lds_barrier();
        read_frags(0, 0, a0, b0);
        static_for<NPART>([&](auto pc) __attribute__((always_inline)) {
            constexpr int p = decltype(pc)::value;
            const int ub = p * nsup / NPART, ue = (p + 1) * nsup / NPART;
            if constexpr (p + 1 < NPART) {
                for (int u = ub; u < ue; u++) superstep(u);
                if constexpr (ACC) {
                    add_c(pc, 2 * DPS * (ue - ub));
                    load_c(p + 1);
                }
            } else {
                for (int u = ub; u < ue - 1; u++) superstep(u);
                last_super();
                if constexpr (ACC) add_c(pc, 2 * DPS * (ue - 1 - ub));
            }
        });
    } else {
    wait_vmcnt_le(3 * DPS + CQ);
    lds_barrier();
    read_frags(0, 0, a0, b0);
    static_for<NPART>([&](auto pc) __attribute__((always_inline)) {
        constexpr int p = decltype(pc)::value;
        const int kb = p * nk / NPART, ke = (p + 1) * nk / NPART;
        if constexpr (p + 1 < NPART) {
            for (int kt = kb; kt < ke; kt++) step(kt);
            if constexpr (ACC) {
                add_c(pc, DPS * (ke - kb));
                load_c(p + 1);
            }
        } else {
            for (int kt = kb; kt < ke - 1; kt++) step(kt);
            last_step();
            if constexpr (ACC) add_c(pc, DPS * (ke - 1 - kb));
        }
    });
    }

    // Epilogue: each 32-row accumulator tile goes through a wave-private LDS area (the ring is free
    // once every wave has passed the barrier) so that every global store writes whole row segments
    // of the wave's FN*128-byte column range: 1 KiB contiguous per instruction instead of 32 rows
    // x 32 bytes.  Row pitch FN*128 + 16 bytes keeps both LDS access patterns conflict-free.
    // The last steps issued clamped copies of the final stage into the ring (never read); every
    // wave waits for its DMA to land (vmcnt(0)) before the barrier, or a late copy could overwrite
    // the C values staged in the same LDS below.
    wait_vmcnt<0>();
    lds_barrier();
    constexpr int PB = FN * 128 + 16;   // LDS row pitch (bytes)
    constexpr int CPR = FN * 8;         // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;       // rows per store instruction
    uint8_t *cst = smem + w * (32 * PB);
    const int sr = lane / CPR, sc = lane % CPR;
    int32_t *cw = C + (size_t)(m0 + wm * 128 + sr) * N + n0 + wn * FN * 32 + 4 * sc;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                *(v4i *)(cst + lcol * PB + 4 * (32 * j + 8 * q + 4 * lgrp)) =
                    v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
#pragma unroll
        for (int t = 0; t < 32 / RPI; t++)
            store_c16(cw + (size_t)(32 * i + RPI * t) * N, *(const v4i *)(cst + (RPI * t + sr) * PB + 16 * sc));
    }
}

// Skinny GEMM, M <= MR rows.  Block = W waves over columns [n0, n0+256) and k rows
// [k0, k0+256); wave w owns rows k0 + RW*w .. +RW-1 (RW = 256/W).  Each lane streams RW/4 x 16
// bytes of B (one 256-byte row slice per 16 lanes, fully coalesced), the wave stages its slice in
// LDS group by group as it arrives, and each lane owns 4 columns: it reads 4 rows' dwords,
// transposes them to k-quads and runs dot4 against the A k-quads (wave-uniform LDS broadcast).
// All loads are unconditional buffer loads issued before the first wait (A's first, since the
// barrier waits for A and loads complete in order).  The W waves' partial sums are reduced in LDS
// and added to C with int32 atomics.  B must fit one buffer resource (K*N < 2^32 bytes).  (W = 8, two waves per SIMD, measured slower: 11.3 vs
// 8.9 us at 8 x 4096 x 4096.)
template <int MR, int W>
__global__ __launch_bounds__(64 * W) void k_gemm_skinny(int M, int N, int K,
                                                       const int8_t *__restrict__ A,
                                                       const int8_t *__restrict__ B,
                                                       int32_t *__restrict__ C)
{
    constexpr int RW = 256 / W;      // k rows per wave
    constexpr int LPL = RW / 4;      // 16-byte loads per lane
    static_assert(W * MR * 256 <= 4 * 64 * 64, "the reduction must fit the B staging area");
    __shared__ __attribute__((aligned(16))) uint32_t Bs[W][RW * 64];  // 64 KB: W x (RW rows x 256 B)
    __shared__ __attribute__((aligned(16))) uint32_t As[MR][64];      // A[m][k0..k0+256) as dwords

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n0 = blockIdx.x * 256, k0 = blockIdx.y * 256;
    // A slice (zero padded) first: the barrier below waits for these loads, and loads complete in
    // order, so A must not queue behind the B slice.
    // Unconditional byte loads through a buffer resource of M*K bytes (rows m >= M read 0); the
    // K tail is zeroed by a select, so every load is issued before any is waited for.
    const rsrc_t ar = buf_rsrc(A, (uint32_t)(M * K));
    static_assert((MR * 64) % (64 * W) == 0, "the A slice is split evenly over the threads");
    constexpr int AJ = MR * 64 / (64 * W);   // A dwords per thread
    uint32_t av[AJ];
#pragma unroll
    for (int j = 0; j < AJ; j++) {
        const int idx = tid + 64 * W * j;
        const int m = idx >> 6, kq = idx & 63;
        const int gk = k0 + 4 * kq;
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int k = gk + e;
            const uint32_t byte = __builtin_amdgcn_raw_buffer_load_b8(ar, (uint32_t)(m * K + min(k, K - 1)), 0, 0);
            v |= (k < K ? byte : 0u) << (8 * e);
        }
        av[j] = v;
    }
    // Then all B loads, so the whole slice is in flight.
    // Unconditional buffer loads: rows past K read 0 (past the resource's K*N bytes); columns past
    // N read the next row's bytes, but those columns are never stored.
    const rsrc_t br = buf_rsrc(B, (uint32_t)((size_t)K * N));
    v4i rb[LPL];
    const int nc = lane & 15;
    const int gn = n0 + 16 * nc;
#pragma unroll
    for (int i = 0; i < LPL; i++) {
        const int gk = k0 + RW * w + 4 * i + (lane >> 4);
        rb[i] = (v4i)__builtin_amdgcn_raw_buffer_load_b128(br, (uint32_t)min((size_t)gk * N + gn, (size_t)K * N), 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the first store
#pragma unroll
    for (int j = 0; j < AJ; j++) {
        const int idx = tid + 64 * W * j;
        As[idx >> 6][idx & 63] = av[j];
    }
    __syncthreads();   // A is in LDS; each wave's B slice is its own, written and read below

    int acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[m][e] = 0;

    // Groups of 16 k-rows: a group goes to LDS as soon as its 4 loads arrive and is consumed at
    // once, so early groups' dot products overlap later groups' loads.  (LDS operations of one
    // wave complete in order, so the wave reads its own rows back without a barrier.)
    const uint32_t *bw = Bs[w];
#pragma unroll
    for (int g = 0; g < LPL / 4; g++) {
#pragma unroll
        for (int i = 4 * g; i < 4 * g + 4; i++) {
            const int row = 4 * i + (lane >> 4);
            *(v4i *)(&Bs[w][row * 64 + 4 * nc]) = rb[i];
        }
#pragma unroll
        for (int kq = 4 * g; kq < 4 * g + 4; kq++) {
            uint32_t o0, o1, o2, o3;
            transpose4x4(bw[(4 * kq + 0) * 64 + lane], bw[(4 * kq + 1) * 64 + lane],
                         bw[(4 * kq + 2) * 64 + lane], bw[(4 * kq + 3) * 64 + lane], o0, o1, o2, o3);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const int a = (int)As[m][(RW / 4) * w + kq];
                acc[m][0] = dot4((int)o0, a, acc[m][0]);
                acc[m][1] = dot4((int)o1, a, acc[m][1]);
                acc[m][2] = dot4((int)o2, a, acc[m][2]);
                acc[m][3] = dot4((int)o3, a, acc[m][3]);
            }
        }
    }
    __syncthreads();

    // Cross-wave reduction through LDS (reuses the B staging area).
    int *red = (int *)&Bs[0][0];  // [W waves][MR][256 columns]
#pragma unroll
    for (int m = 0; m < MR; m++)
        *(v4i *)(&red[(w * MR + m) * 256 + 4 * lane]) = v4i{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
    __syncthreads();
    for (int t = tid; t < MR * 256; t += 64 * W) {
        const int m = t >> 8, c = t & 255;
        const int col = n0 + c;
        if (m < M && col < N) {
            int sum = 0;
#pragma unroll
            for (int v = 0; v < W; v++) sum += red[(v * MR + m) * 256 + c];
            atomicAdd(&C[(size_t)m * N + col], sum);
        }
    }
}

// Skinny GEMM on the matrix cores: M <= 16 rows, N % 128 == 0, K % 512 == 0.  Block = 4 waves over
// columns [n0, n0+128) and k rows [k0, k0+512) (split-K over blockIdx.y).  The block's B slab
// (512 k-rows x 128 bytes, 64 KiB) reaches LDS by global->LDS DMA in eight 64-row chunks, the
// 16-byte chunk c of k-row k stored at position c ^ 2((k >> 1) & 3) ^ ((k >> 4) & 1), so that each
// transposing read below serves 32 lanes from 32 distinct banks; each chunk is multiplied as soon as
// every wave's part of it has landed.  Wave w owns columns n0 + 32w .. +31 (two 16-column tiles)
// and runs v_mfma_i32_16x16x64_i8 with A = the token rows (lane l: row l % 16 (zero from M), bytes
// 16(l / 16) .. +15 of the 64-k chunk; the rows' 512-byte slice is staged in LDS too) and B = 64 k x
// 16 columns (lane l: column l % 16, the same 16 k), two ds_read_b64_tr_b8 each (lane q of a 16-lane
// group receives column q of an 8 x 16 byte block).  The accumulator holds C[4(l / 16) + r][column
// l % 16]; the block's partial sums are added into C with int32 atomics (exact, order independent).
X100_DEV int skm_swz(int k, int c) { return c ^ (2 * ((k >> 1) & 3)) ^ ((k >> 4) & 1); }


__global__ __launch_bounds__(256) void k_gemm_skinny_mfma(int M, int N, int K, const int8_t *__restrict__ A,
                                                         const int8_t *__restrict__ B, int32_t *__restrict__ C)
{
    __shared__ __attribute__((aligned(16))) uint8_t Bs[512 * 128];
    __shared__ __attribute__((aligned(16))) uint8_t As[16 * 512];   // token rows, chunk c of row q at c ^ (q & 15)
    const int lane = threadIdx.x & 63, w = wave_id(), g = lane >> 4, q = lane & 15;
    const int n0 = blockIdx.x * 128, k0 = blockIdx.y * 512;
    const uint32_t sb = lds_addr(Bs), sa = lds_addr(As);

    // Every wave's DMA ops, oldest first: its two A ops (rows 4w .. 4w+3, clamped to M - 1; rows from
    // M are zeroed in registers), then its 16 B ops: op i = 4t + w (t = 0..15) copies k-rows
    // 8i .. 8i+7 (chunk t / 2 of 64 rows); lane L lands at row 8i + L/8, position L%8 and fetches the
    // chunk stored there.
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int i = 2 * w + t, row = 2 * i + (lane >> 5);
        dma16v(A + (size_t)min(row, M - 1) * K + k0 + 16 * ((lane & 31) ^ (row & 15)),
               __builtin_amdgcn_readfirstlane(sa + (uint32_t)(1024 * i)));
    }
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const int i = 4 * t + w, kr = 8 * i + (lane >> 3);
        dma16v(B + (size_t)(k0 + kr) * N + n0 + 16 * skm_swz(kr, lane & 7),
               __builtin_amdgcn_readfirstlane(sb + (uint32_t)(1024 * i)));
    }

    v4i acc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
    const int r8 = q >> 1, h8 = q & 1;
    static_for<8>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        wait_vmcnt<2 * (7 - j)>();   // this wave's A ops and its two B ops of chunk j have landed
        lds_barrier();                // and every other wave's
        v4i a = *(const v4i *)(As + q * 512 + 16 * ((4 * j + g) ^ q));
        a = q < M ? a : v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int c = 2 * w + t;   // the tile's 16-byte column chunk
            const int kr0 = 64 * j + 16 * g + r8, kr1 = kr0 + 8;
            const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_v2i *)(const lds_u8 *)(Bs + kr0 * 128 + 16 * skm_swz(kr0, c) + 8 * h8));
            const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_v2i *)(const lds_u8 *)(Bs + kr1 * 128 + 16 * skm_swz(kr1, c) + 8 * h8));
            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, v4i{lo.x, lo.y, hi.x, hi.y}, acc[t], 0, 0, 0);
        }
    });
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * g + r;
            if (m < M) atomicAdd(&C[(size_t)m * N + n0 + 32 * w + 16 * t + q], acc[t][r]);
        }
}

// Generic fallback: 64x64 tile, 256 threads (4x4 outputs each), 32-deep byte tiles in LDS.
// ACC: C += A.B; otherwise C = A.B (C not read).
template <bool ACC>
__global__ __launch_bounds__(256) void k_gemm_generic(int M, int N, int K, const int8_t *__restrict__ A,
                                                      const int8_t *__restrict__ B,
                                                      int32_t *__restrict__ C)
{
    __shared__ int As[64][33];
    __shared__ int Bs[32][65];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    int acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 32) {
        for (int idx = tid; idx < 64 * 32; idx += 256) {
            int r = idx >> 5, c = idx & 31;
            int gm = m0 + r, gk = k0 + c;
            As[r][c] = (gm < M && gk < K) ? (int)A[(size_t)gm * K + gk] : 0;
            int kr = idx >> 6, nc2 = idx & 63;
            int gk2 = k0 + kr, gn = n0 + nc2;
            Bs[kr][nc2] = (gk2 < K && gn < N) ? (int)B[(size_t)gk2 * N + gn] : 0;
        }
        __syncthreads();
        for (int k = 0; k < 32; k++) {
            int a[4], b[4];
            for (int i = 0; i < 4; i++) a[i] = As[ty * 4 + i][k];
            for (int j = 0; j < 4; j++) b[j] = Bs[k][tx * 4 + j];
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 4; j++) acc[i][j] += a[i] * b[j];
        }
        __syncthreads();
    }
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) {
            int gm = m0 + ty * 4 + i, gn = n0 + tx * 4 + j;
            if (gm < M && gn < N) C[(size_t)gm * N + gn] = ACC ? C[(size_t)gm * N + gn] + acc[i][j] : acc[i][j];
        }
}

template <int FM, int FN, int WM, int WN, bool ACC>
hipError_t launch_mfma_acc(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C,
                           hipStream_t s)
{
    constexpr int BM = WM * FM * 32, BN = WN * FN * 32;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const bool edge = (M % BM) || (N % BN) || (K % BK);
    if (edge)
        hipLaunchKernelGGL((k_gemm_mfma<FM, FN, WM, WN, true, ACC>), dim3(tiles_m * tiles_n),
                           dim3(WM * WN * 64), 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_mfma<FM, FN, WM, WN, false, ACC>), dim3(tiles_m * tiles_n),
                           dim3(WM * WN * 64), 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    return hipGetLastError();
}

template <int FM, int FN, int WM, int WN>
hipError_t launch_mfma(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C, hipStream_t s,
                       bool acc)
{
    return acc ? launch_mfma_acc<FM, FN, WM, WN, true>(M, N, K, A, B, C, s)
               : launch_mfma_acc<FM, FN, WM, WN, false>(M, N, K, A, B, C, s);
}

// The 256x256 tile kernel k_gemm_big<NW, SUPER, ACC> (M, N multiples of 256, K % 64 == 0,
// K >= 512); superstages when K / 64 is a multiple of 8 (the K shapes that path is tested on).
template <int NW>
hipError_t launch_big(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C, hipStream_t s, bool acc)
{
    const int tiles_m = M / 256, tiles_n = N / 256;
    const dim3 grid(tiles_m * tiles_n), block(NW * 64);
    const bool super = (K / BK) % 8 == 0;
    if (super && acc)
        hipLaunchKernelGGL((k_gemm_big<NW, 2, true>), grid, block, 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    else if (super)
        hipLaunchKernelGGL((k_gemm_big<NW, 2, false>), grid, block, 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    else if (acc)
        hipLaunchKernelGGL((k_gemm_big<NW, 1, true>), grid, block, 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_big<NW, 1, false>), grid, block, 0, s, M, N, K, A, B, C, tiles_m, tiles_n);
    return hipGetLastError();
}

// C = 0 for the overwrite form (C = A*B): 16-byte stores from the first 16-byte boundary, single
// int32 stores before it and for the tail (a kernel rather than hipMemsetAsync, so that a caller
// can capture it in a graph).
__global__ __launch_bounds__(256) void k_zero_i32(int32_t *__restrict__ C, size_t n)
{
    const size_t head = min(n, (size_t)((16 - ((uintptr_t)C & 15)) & 15) / 4);
    const size_t nv = (n - head) / 4;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
    v4i *cv = (v4i *)(C + head);
    for (size_t i = t; i < nv; i += stride) cv[i] = v4i{0, 0, 0, 0};
    if (t < head) C[t] = 0;
    for (size_t i = head + 4 * nv + t; i < n; i += stride) C[i] = 0;
}

}  // namespace

hipError_t x100_zero_i32_launch(int32_t *C, size_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    const size_t blocks = min((n / 4 + 255) / 256 + 1, (size_t)4096);
    hipLaunchKernelGGL(k_zero_i32, dim3((unsigned)blocks), dim3(256), 0, s, C, n);
    return hipGetLastError();
}

// Kernel selection.  acc: C += A.B; otherwise C = A.B (the tile kernels never read C; the
// split-K skinny kernels add partial sums with atomics, so their C is cleared first).  Returns the
// HIP launch status.
hipError_t x100_gemm_i8_launch(int M, int N, int K, const int8_t *A, const int8_t *B, int32_t *C,
                               hipStream_t s, int variant, bool acc)
{
    const bool aligned = (K % 16 == 0) && (N % 16 == 0) && (((uintptr_t)A & 15) == 0) &&
                         (((uintptr_t)B & 15) == 0) && (((uintptr_t)C & 15) == 0);
    if (variant == X100_GEMM_AUTO) {
        if (!aligned)
            variant = X100_GEMM_GENERIC;
        else if (M <= 16 && (size_t)K * N < ((size_t)1 << 32))   // B must fit one buffer resource
            variant = X100_GEMM_SKINNY;
        // Tile by output size, measured at K = 1024-4096 (graph replay, us): 256x256 tiles from
        // 4M outputs (2048^2 x 4096: 50.3 vs 52.6 with 128x128), 64x64 from 1M (1024^2 x 4096:
        // 27.3 vs 39.9 / 45.2), 32x32 below (256^3: 3.5 vs 5.7; 512^3: 4.9 vs 7.9).  Smaller tiles
        // put enough blocks on the 256 CUs when the product has few 256x256 tiles.
        else if ((long)M * N >= 4L * 1024L * 1024L)
            variant = X100_GEMM_TILE256;
        else if ((long)M * N >= 1024L * 1024L)
            variant = X100_GEMM_TILE64;
        else
            variant = X100_GEMM_TILE32;
    }
    if (!aligned && variant != X100_GEMM_GENERIC) return hipErrorInvalidValue;
    switch (variant) {
    case X100_GEMM_TILE256:
        // Full 256x256 tiles only; other shapes use the 128x128 tile with edge guards.
        if (M % 256 || N % 256 || K % BK || K < 512) return launch_mfma<2, 2, 2, 2>(M, N, K, A, B, C, s, acc);
        return launch_big<8>(M, N, K, A, B, C, s, acc);
    case X100_GEMM_TILE256_W4:
        if (M % 256 || N % 256 || K % BK || K < 512) return launch_mfma<2, 2, 2, 2>(M, N, K, A, B, C, s, acc);
        return launch_big<4>(M, N, K, A, B, C, s, acc);
    case X100_GEMM_TILE128: return launch_mfma<2, 2, 2, 2>(M, N, K, A, B, C, s, acc);
    case X100_GEMM_TILE64: return launch_mfma<1, 1, 2, 2>(M, N, K, A, B, C, s, acc);
    case X100_GEMM_TILE32: return launch_mfma<1, 1, 1, 1>(M, N, K, A, B, C, s, acc);
    case X100_GEMM_SKINNY: {
        if (M > 16 || (size_t)K * N >= ((size_t)1 << 32)) return hipErrorInvalidValue;
        if (!acc) {
            const hipError_t e = x100_zero_i32_launch(C, (size_t)M * N, s);
            if (e != hipSuccess) return e;
        }
        dim3 grid((N + 255) / 256, (K + 255) / 256);
        if (N % 128 == 0 && K % 512 == 0) {   // whole 512 x 128 slabs: the matrix-core kernel
            hipLaunchKernelGGL(k_gemm_skinny_mfma, dim3(N / 128, K / 512), dim3(256), 0, s, M, N, K, A, B, C);
            return hipGetLastError();
        }
        if (M <= 8)
            hipLaunchKernelGGL((k_gemm_skinny<8, 4>), grid, dim3(256), 0, s, M, N, K, A, B, C);
        else
            hipLaunchKernelGGL((k_gemm_skinny<16, 4>), grid, dim3(256), 0, s, M, N, K, A, B, C);
        return hipGetLastError();
    }
    case X100_GEMM_GENERIC: {
        dim3 grid((N + 63) / 64, (M + 63) / 64);
        if (acc)
            hipLaunchKernelGGL(k_gemm_generic<true>, grid, dim3(256), 0, s, M, N, K, A, B, C);
        else
            hipLaunchKernelGGL(k_gemm_generic<false>, grid, dim3(256), 0, s, M, N, K, A, B, C);
        return hipGetLastError();
    }
    }
    return hipErrorInvalidValue;
}
