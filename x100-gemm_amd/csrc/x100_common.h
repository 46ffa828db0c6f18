// Shared device helpers for the gfx950 kernels of libx100hip.
//
// All kernels are compiled with -ffp-contract=off: every fp32 expression is rounded after each
// operation exactly as written, which is what lets the MoE path reproduce the scalar oracle's
// intermediate activations bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

#define X100_DEV __device__ __forceinline__

// GGUF type ids (bench/gguf_dump.c:12-13 of the reference).
enum { X100_Q4_0 = 2, X100_Q8_0 = 8, X100_Q3_K = 11, X100_Q4_K = 12, X100_Q5_K = 13, X100_Q6_K = 14 };

// fp16 bits -> fp32 (exact).
X100_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16 bits as the reference's f32_to_f16 (qwen_moe_hp.c:71-79) converts, which every
// fp16 scale of its Q8_0 quantizer goes through: the 13 low mantissa bits are dropped (a normal
// result is the magnitude truncated, never rounded up), results below the normal range are
// truncated into the subnormal field and below 2^-24 to a signed zero, and exponents past the
// fp16 range (|f| >= 2^16, inf, NaN) give a signed infinity.  Selects only, no branches.
X100_DEV uint16_t f2h_trunc(float f)
{
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e16 = (int)((x >> 23) & 0xffu) - 112;
    const uint32_t frac = x & 0x7fffffu;
    const uint32_t normal = sign | ((uint32_t)e16 << 10) | (frac >> 13);
    const uint32_t sub = sign | ((frac | 0x800000u) >> min(max(14 - e16, 0), 31));
    uint32_t r = e16 > 0 ? normal : (e16 < -10 ? sign : sub);
    r = e16 >= 31 ? (sign | 0x7c00u) : r;
    return (uint16_t)r;
}

// 4-way int8 dot product with int32 accumulate: acc + sum_i a.b[i]*b.b[i] (signed bytes).
X100_DEV int dot4(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

// v_perm_b32: result byte k = byte sel.byte[k] of the 8-byte value (hi:lo).
X100_DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4x4 byte transpose: r[i] holds 4 bytes (columns 0..3) of row i; o[c] receives column c as
// 4 bytes (rows 0..3, row 0 in the low byte).
X100_DEV void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t &o0,
                           uint32_t &o1, uint32_t &o2, uint32_t &o3)
{
    uint32_t x01l = perm(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
    uint32_t x01h = perm(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
    uint32_t x23l = perm(r3, r2, 0x05010400u);  // r2.b0 r3.b0 r2.b1 r3.b1
    uint32_t x23h = perm(r3, r2, 0x07030602u);  // r2.b2 r3.b2 r2.b3 r3.b3
    o0 = perm(x23l, x01l, 0x05040100u);         // r0.b0 r1.b0 r2.b0 r3.b0
    o1 = perm(x23l, x01l, 0x07060302u);         // r0.b1 r1.b1 r2.b1 r3.b1
    o2 = perm(x23h, x01h, 0x05040100u);
    o3 = perm(x23h, x01h, 0x07060302u);
}

// Index of the calling wave in its block, as a wave-uniform (scalar) value: addresses derived from
// it (buffer resources, M0) stay in scalar registers.
X100_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// The value of lane l^32 / l^16 (what __shfl_xor(v, 32 / 16, 64) returns), in VALU instructions
// instead of an LDS permute: v_permlane32_swap / v_permlane16_swap with both operands v leave the
// lower row (half) of each pair in the first result and the upper one in the second, and the lane
// takes the one that is not its own.
X100_DEV uint32_t xor32_u(uint32_t v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
}
X100_DEV uint32_t xor16_u(uint32_t v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
}
X100_DEV float xor32_f(float v) { return __uint_as_float(xor32_u(__float_as_uint(v))); }
X100_DEV float xor16_f(float v) { return __uint_as_float(xor16_u(__float_as_uint(v))); }
X100_DEV int xor32_i(int v) { return (int)xor32_u((uint32_t)v); }
X100_DEV int xor16_i(int v) { return (int)xor16_u((uint32_t)v); }


// ------------------------------------------------------------------------------------------------
// Lane reductions with DPP (data-parallel primitives: a VALU operand read from another lane of
// the same row of 16, a few cycles) instead of ds_bpermute shuffles.
//   quad_perm 0xB1 = lanes [1,0,3,2] (xor 1), 0x4E = [2,3,0,1] (xor 2);
//   row_half_mirror 0x141: lane i <- lane 7-i within each group of 8;
//   row_shr:n 0x110+n; row_bcast:15 0x142 / row_bcast:31 0x143 (lane 15 / 31 of the previous
//   row(s) into the rows enabled by the row mask).
// A lane whose source lane is invalid (row_shr at the start of a row) or whose row is masked off
// receives `old` instead: v itself for a maximum, 0 for a sum.
// ------------------------------------------------------------------------------------------------
template <int CTRL, int ROWM = 0xf, int BANKM = 0xf>
X100_DEV int dpp_i(int old, int v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWM, BANKM, false);
}
template <int CTRL, int ROWM = 0xf, int BANKM = 0xf>
X100_DEV float dpp_f(float old, float v)
{
    return __int_as_float(dpp_i<CTRL, ROWM, BANKM>(__float_as_int(old), __float_as_int(v)));
}
// Sum / max over each aligned group of 4 or 8 lanes, result in every lane of the group.
X100_DEV int sum4_i(int v)
{
    v += dpp_i<0xB1>(0, v);
    v += dpp_i<0x4E>(0, v);
    return v;
}
X100_DEV int sum8_i(int v)
{
    v = sum4_i(v);
    v += dpp_i<0x141>(0, v);
    return v;
}
X100_DEV float max8_f(float v)
{
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    return v;
}
// Maximum over the 64 lanes, returned wave-uniform (prefix maximum into lane 63, then readlane).
X100_DEV float wave_max_u(float v)
{
    v = fmaxf(v, dpp_f<0x111>(v, v));
    v = fmaxf(v, dpp_f<0x112>(v, v));
    v = fmaxf(v, dpp_f<0x114>(v, v));
    v = fmaxf(v, dpp_f<0x118>(v, v));
    v = fmaxf(v, dpp_f<0x142, 0xa>(v, v));
    v = fmaxf(v, dpp_f<0x143, 0xc>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Integer maximum over the 64 lanes, wave-uniform.  The "old" operand is INT_MIN, the identity
// of max, so each step compiles to one v_max_i32_dpp.
X100_DEV int wave_max_iu(int v)
{
    v = max(v, dpp_i<0x111>(INT_MIN, v));
    v = max(v, dpp_i<0x112>(INT_MIN, v));
    v = max(v, dpp_i<0x114>(INT_MIN, v));
    v = max(v, dpp_i<0x118>(INT_MIN, v));
    v = max(v, dpp_i<0x142, 0xa>(INT_MIN, v));
    v = max(v, dpp_i<0x143, 0xc>(INT_MIN, v));
    return __builtin_amdgcn_readlane(v, 63);
}
// Sum over the 64 lanes in xor-butterfly order (lane l adds lane l^32, then l^16, l^8, l^4, l^2,
// l^1): the value six __shfl_xor steps give, bit for bit.  The l^32 and l^16 partners come from
// permlane swaps.  After the first two levels a lane's value depends only on l mod 16, after the
// third only on l mod 8, so row_ror:8 and row_ror:4 (rotations within a row of 16) deliver the l^8
// and l^4 partners' values; quad_perm does l^2, l^1.
X100_DEV float wave_sum_bfly_f(float s)
{
    s += xor32_f(s);
    s += xor16_f(s);
    s += dpp_f<0x128>(0.0f, s);
    s += dpp_f<0x124>(0.0f, s);
    s += dpp_f<0x4E>(0.0f, s);
    s += dpp_f<0xB1>(0.0f, s);
    return s;
}
// Sum over the 64 lanes, wave-uniform: prefix sum of rows (row_shr 1, 2, 4, 8), then rows
// combined into lane 63.  For integers, or floats whose summation order is not prescribed.
X100_DEV int wave_sum_u(int v)
{
    v += dpp_i<0x111>(0, v);
    v += dpp_i<0x112>(0, v);
    v += dpp_i<0x114>(0, v);
    v += dpp_i<0x118>(0, v);
    v += dpp_i<0x142, 0xa>(0, v);
    v += dpp_i<0x143, 0xc>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}
X100_DEV float wave_sum_uf(float v)
{
    v += dpp_f<0x111>(0.0f, v);
    v += dpp_f<0x112>(0.0f, v);
    v += dpp_f<0x114>(0.0f, v);
    v += dpp_f<0x118>(0.0f, v);
    v += dpp_f<0x142, 0xa>(0.0f, v);
    v += dpp_f<0x143, 0xc>(0.0f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// wave_sum_uf of N values at once, each step applied to all of them so that their DPP chains
// interleave (each value's additions in the same order as wave_sum_uf).
template <int N>
X100_DEV void wave_sum_uf_n(float (&v)[N])
{
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x111>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x112>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x114>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x118>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x142, 0xa>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f<0x143, 0xc>(0.0f, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), 63));
}

// Device-side Q8 activation formats (kept in LDS or a workspace; internal to the library).
//   Q8_0 (per 32): fp16 d, int8 q[32], int sum(q)     -- quantize_q8_0_native rounding
//   Q8_K (per 256): fp32 d, int8 q[256], int bsum[16] -- pack_A_q3k rounding
// Quantize one 32-element block held by one thread (values v[0..31]).
X100_DEV float q8_0_scale(float amax) { return amax / 127.0f; }
X100_DEV int clamp_i8(int q) { return q > 127 ? 127 : (q < -128 ? -128 : q); }

// Raw buffer resource over [p, p + bytes): loads at byte offsets >= bytes return 0 instead of
// touching memory, so bounds-checked loads need no branch (word 3 = gfx9 raw buffer format).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
X100_DEV rsrc_t buf_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
X100_DEV float4 buf_load_f4(rsrc_t r, uint32_t byte_off)
{
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
}

// Asynchronous global -> LDS copy of 1 KiB per wave (global_load_lds_dwordx4): lane l copies the
// 16 bytes at its own src to lds_base + 16*l.  lds_base must be the same for the whole wave.  The
// compiler counts these loads like any other (a __syncthreads() waits for them).
X100_DEV void dma_1k(const void *src, void *lds_base)
{
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
}

// LDS byte address of a pointer into LDS (the M0 operand of the DMA below).
X100_DEV uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// The same 16-byte-per-lane global -> LDS DMA from a per-lane address, issued from inline asm: the
// compiler does not count it, so it inserts no wait for it and the kernel waits for it itself
// (s_waitcnt vmcnt; each wave's operations complete in issue order).  lds_base is wave-uniform.
X100_DEV void dma16v(const void *src, uint32_t lds_base)
{
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}

// ------------------------------------------------------------------------------------------------
// Activation quantizers for a 256-thread block.  The M x K fp32 rows are read as float4 (float4
// f = c0 + tid + 256*i holds elements 4f .. 4f+3 of the flattened rows) in chunks of XPT float4
// per thread (NT threads per block): x_load issues a chunk's loads (through a buffer resource of M*K*4 bytes, so
// elements past the end read as 0), the *_from_regs functions quantize the chunk into LDS.
// Kernels issue chunk 0 before their weight loads so that it arrives while the weights are still
// in flight.
//   Q8_0 (quantize_q8_0_native rounding): a 32-element block is 8 consecutive threads.
//   Q8_K (pack_A_q3k rounding): a 256-element block is one wave (64 threads).
// ------------------------------------------------------------------------------------------------
template <int XPT, int NT = 256>
X100_DEV void x_load(rsrc_t xr, int c0, float4 (&v)[XPT])
{
#pragma unroll
    for (int i = 0; i < XPT; i++) v[i] = buf_load_f4(xr, (uint32_t)(c0 + threadIdx.x + NT * i) * 16u);
}

// Branch-free stores (so the unrolled iterations can be interleaved by the scheduler): blocks past
// the end go to the spare slot (index M*nb / M*nsb) that the LDS layout provides, and values that
// several lanes hold (d, sum) are stored by all of them.
// F16D: the block scale is stored as fp16 by the reference's truncating conversion
// (quantize_q8_0_native, qwen_moe_hp.c:408-414) or kept in fp32 (pack_A_i8,
// qwen_moe_q3k.c:420-427); the q values are the same either way (they use the fp32 scale).
// OFS: also store -8 * (sum of the block's q), the offset term of a Q4_0 dot ((u - 8).q =
// u.q - 8 * sum q for nibbles u), so that the dot starts from it; the int8 path needs no sums.
//
// The arithmetic is the reference's (d = amax / 127.0f, inv = 1.0f / d, q = lrintf(x * inv), fp16 d
// by truncation), computed without IEEE division and without a clamp:
// * d by one product with RN(1/127) and an FMA correction, inv by v_rcp_f32 and one Newton step.
//   For every amax in [1e-6, FLT_MAX] (all 1,241,106,499 floats) both equal the correctly
//   rounded quotients, checked exhaustively on gfx950.
// * q: x * inv is rounded to float, then 1.5 * 2^23 is added, which rounds it to an integer with
//   ties to even (rintf); the sum's low byte is q modulo 256.  |x * inv| <= 127 * (1 + 2^-23), so
//   q is in [-127, 127] and the reference's clamp never applies.
// * fp16 truncation of d (> 0, finite): the top 10 mantissa bits from 2^-14 up, multiples of
//   2^-24 below, infinity from 65536 (equal to f32_to_f16 then f16_to_f32 for every positive
//   float).
// Non-finite activations give unspecified bytes (the reference's lrintf of NaN is
// implementation-defined too).
X100_DEV float div127_rn(float a)
{
    const float c = 0x1.020408p-7f;   // RN(1/127)
    const float q0 = a * c;
    const float r = __builtin_fmaf(-q0, 127.0f, a);
    return __builtin_fmaf(r, c, q0);
}
X100_DEV float rcp_rn(float d)
{
    const float y0 = __builtin_amdgcn_rcpf(d);
    const float e = __builtin_fmaf(-d, y0, 1.0f);
    return __builtin_fmaf(e, y0, y0);
}
// 1.0f / d correctly rounded for every d in [0, 2^126], and 0 for d = 0 (the Q8_K quantizers'
// reciprocal, whose amax has no floor).  rcp_rn is exact on [2^-126, 2^126] (checked on gfx950
// for every float there; it fails on subnormals).  A subnormal d is scaled by 2^64 into that range
// and the reciprocal scaled back: both scalings are exact, and the product overflows to infinity
// exactly when 1/d rounds to infinity, so the result is RN(1/d) there too.
X100_DEV float rcp_rn_any(float d)
{
    const bool sub = d < 0x1p-126f;
    const float r = rcp_rn(sub ? d * 0x1p64f : d);
    return d == 0.0f ? 0.0f : (sub ? r * 0x1p64f : r);
}
X100_DEV float f16_trunc_pos(float d)
{
    const float nrm = __uint_as_float(__float_as_uint(d) & 0xffffe000u);
    const float sub = __builtin_truncf(d * 0x1p24f) * 0x1p-24f;
    const float r = d >= 0x1p-14f ? nrm : sub;
    return d >= 65536.0f ? __builtin_inff() : r;
}
template <int XPT, int NT = 256, bool F16D = true, bool OFS = true>
X100_DEV void q8_0_from_regs(const float4 (&v)[XPT], int c0, int total4, int K, int8_t *xlo,
                             int8_t *xhi, float *xd, int *xs)
{
    (void)K;   // rows are contiguous and K % 32 == 0: element e is in 32-block e / 32
    constexpr float RND = 0x1.8p23f;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int f = c0 + threadIdx.x + NT * i;
        const float a = max8_f(fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        const float amax = fmaxf(a, 1e-6f);
        const float d = div127_rn(amax);
        const float inv = rcp_rn(d);
        const float p0 = v[i].x * inv, p1 = v[i].y * inv, p2 = v[i].z * inv, p3 = v[i].w * inv;
        const uint32_t t0 = __float_as_uint(p0 + RND), t1 = __float_as_uint(p1 + RND);
        const uint32_t t2 = __float_as_uint(p2 + RND), t3 = __float_as_uint(p3 + RND);
        const uint32_t packed = perm(t1, t0, 0x0c0c0400u) | perm(t3, t2, 0x04000c0cu);
        const int pos = 4 * (f & 7);
        const int b = f < total4 ? f >> 3 : total4 >> 3;   // spare block past the end
        int8_t *dst = pos < 16 ? xlo + b * 16 + pos : xhi + b * 16 + (pos - 16);
        *(uint32_t *)dst = packed;
        xd[b] = F16D ? f16_trunc_pos(d) : d;   // the 8 lanes of a block hold the same d and sum
        if constexpr (OFS) xs[b] = -8 * sum8_i(dot4((int)packed, 0x01010101, 0));
    }
}

// Quantize one 256-element block to Q8_K with one wave (the operations of pack_A_q3k,
// qwen_moe_q3k.c:612-624): v is the lane's float4 (elements 4*lane .. 4*lane+3); writes q[256],
// the 16 sums bs[16] and the scale *dout.
X100_DEV void q8_K_wave(const float4 v, int8_t *qs, int *bs, float *dout)
{
    const int lane = threadIdx.x & 63;
    const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    const float amax = wave_max_u(a);
    const float d = div127_rn(amax);
    const float rep = rcp_rn_any(d);
    const int q0 = clamp_i8((int)roundf(v.x * rep)), q1 = clamp_i8((int)roundf(v.y * rep));
    const int q2 = clamp_i8((int)roundf(v.z * rep)), q3 = clamp_i8((int)roundf(v.w * rep));
    ((uint32_t *)qs)[lane] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                             ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
    const int s = sum4_i(q0 + q1 + q2 + q3);
    bs[lane >> 2] = s;   // the 4 lanes of a 16-group hold the same sum (no branch)
    *dout = d;           // d is wave-uniform
}

template <int XPT, int NT = 256>
X100_DEV void q8_K_from_regs(const float4 (&v)[XPT], int c0, int total4, int8_t *xq, int *xbs, float *xd)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int f = c0 + threadIdx.x + NT * i;
        const float a = fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
        const float amax = wave_max_u(a);
        const float d = div127_rn(amax);
        const float rep = rcp_rn_any(d);
        const int q0 = clamp_i8((int)roundf(v[i].x * rep)), q1 = clamp_i8((int)roundf(v[i].y * rep));
        const int q2 = clamp_i8((int)roundf(v[i].z * rep)), q3 = clamp_i8((int)roundf(v[i].w * rep));
        const int s = sum4_i(q0 + q1 + q2 + q3);
        // flattened (row, super-block) index, uniform per wave (total4 is a multiple of 64); the
        // spare block total4/64 takes waves past the end
        const int blk = min(f, total4) / 64;
        ((uint32_t *)(xq + blk * 256))[lane] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                               ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
        xbs[blk * 16 + (lane >> 2)] = s;   // the 4 lanes of a 16-group hold the same sum
        xd[blk] = d;                       // d is wave-uniform
    }
}

// ------------------------------------------------------------------------------------------------
// Q8_K records of 256 activations (the GEMV and the MoE block): q[256] int8 | s16[16] (int sums
// of q per 16) | s32[8] (per 32) | d (fp32 scale), 368 bytes.  Record q = m * nsb + sb of an
// M x K row-major activation holds elements m*K + 256sb .. +255.
// ------------------------------------------------------------------------------------------------
constexpr int KR_S16 = 256, KR_S32 = 320, KR_D = 352, KREC = 368;

// n / d for n, d < 2^16 with m = ceil(2^32 / d) precomputed on the host (exact in that range:
// n * (m - 2^32 / d) / 2^32 < n / 2^32 < 1 / d); d = 1 is passed through.
X100_DEV uint32_t udiv16(uint32_t n, uint32_t d, uint32_t m) { return d == 1 ? n : __umulhi(n, m); }
inline uint32_t udiv16_magic(uint32_t d) { return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + d - 1) / d); }
// roundf(v) (half away from zero) for |v| < 2^23: trunc(v + copysign(0.5 - 2^-25, v)) with the add
// rounded to nearest even.  Below a tie the sum stays under the next integer (its distance to it
// exceeds half an ulp there), at or above a tie it reaches it; checked against roundf for every
// float with |v| <= 128.
X100_DEV int round_away(float v) { return (int)(v + __builtin_copysignf(0x1.fffffep-2f, v)); }

// Q8_K records of x, four per wave pass: lane l works on record q = qb + l/16 (q = m*nsb + sb:
// elements m*K + 256sb ..), elements 16(l%16) .. +15, with the operations of pack_A_q3k
// (qwen_moe_q3k.c:612-624): amax over the record, d = amax/127, reciprocal 1/d (0 for d = 0),
// q = roundf(x * (1/d)) clamped to [-128, 127], plus the sums of q per 16 and per 32 elements.
// Records past nq read zeros and are not stored.
X100_DEV void q8k_load(rsrc_t xr, int K, int nsb, uint32_t mnsb, int nq, int qb, float4 (&v)[4])
{
    const int lane = threadIdx.x & 63, q = qb + (lane >> 4);
    const int m = (int)udiv16((uint32_t)q, (uint32_t)nsb, mnsb), sb = q - m * nsb;
    const uint32_t base = q < nq ? (uint32_t)(m * K + sb * 256 + 16 * (lane & 15)) * 4u : 0xffffff00u;
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = buf_load_f4(xr, base + 16u * c);
}
X100_DEV void q8k_quant(const float4 (&v)[4], int nq, int qb, uint8_t *recs)
{
    const int lane = threadIdx.x & 63, i = lane & 15, q = qb + (lane >> 4);
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++)
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v[c].x), fabsf(v[c].y)), fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
    // maximum over the record's 16 lanes, in every one of them (xor 1, xor 2, mirror in 8, mirror in 16)
    a = fmaxf(a, dpp_f<0xB1>(a, a));
    a = fmaxf(a, dpp_f<0x4E>(a, a));
    a = fmaxf(a, dpp_f<0x141>(a, a));
    a = fmaxf(a, dpp_f<0x140>(a, a));
    const float d = div127_rn(a);
    const float rep = rcp_rn_any(d);
    uint32_t pk[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int q0 = clamp_i8(round_away(v[c].x * rep)), q1 = clamp_i8(round_away(v[c].y * rep));
        const int q2 = clamp_i8(round_away(v[c].z * rep)), q3 = clamp_i8(round_away(v[c].w * rep));
        pk[c] = perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u) | (perm((uint32_t)q3, (uint32_t)q2, 0x0c0c0400u) << 16);
    }
    int s16 = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) s16 = dot4((int)pk[c], 0x01010101, s16);
    const int s32 = s16 + dpp_i<0xB1>(0, s16);   // + the neighbouring 16 elements
    if (q < nq) {
        uint8_t *rec = recs + (size_t)q * KREC;
        *(v4u *)(rec + 16 * i) = v4u{pk[0], pk[1], pk[2], pk[3]};
        ((int *)(rec + KR_S16))[i] = s16;
        ((int *)(rec + KR_S32))[i >> 1] = s32;   // the two lanes of a pair store the same sum
        if (i == 0) *(float *)(rec + KR_D) = d;
    }
}


// ------------------------------------------------------------------------------------------------
// Q4_K x Q8_K on half a super-block: the lane holds qs bytes 64h .. 64h+63 of a Q4_K block as four
// 16-byte planes (plane c: low nibbles of sub-block 4h + 2(c/2), high nibbles of 4h + 2(c/2) + 1,
// elements 16(c%2) .. +16), i.e. sub-blocks 4h .. 4h+3 = elements 128h .. 128h+127, and the 6-bit
// (sc, m) of those four sub-blocks; the unit's other half is the neighbouring lane (lane ^ 1).
// ------------------------------------------------------------------------------------------------
struct Q4kHalf {
    int lo[4][4], hi[4][4];   // [plane][dword] nibbles as bytes
    int sc[4], mn[4];         // 6-bit scale and min of sub-blocks 4h + jj
};
X100_DEV void q4k_unpack(const v4i (&qv)[4], Q4kHalf &u)
{
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            u.lo[c][t] = qv[c][t] & 0x0F0F0F0F;
            u.hi[c][t] = (qv[c][t] >> 4) & 0x0F0F0F0F;
        }
}
// get_scale_min_k4 (repack.cpp:222-233) of sub-blocks 4h .. 4h+3 from the GGUF header dwords
// (hdr[1..3] = the 12 scale bytes s): j < 4 takes s[j] & 63 and s[j+4] & 63; j >= 4 takes
// (s[j+4] & 15) | (s[j-4] >> 6) << 4 and (s[j+4] >> 4) | (s[j] >> 6) << 4, four bytes at a time.
X100_DEV void q4k_scales_gguf(const v4i &hdr, int h, Q4kHalf &u)
{
    const uint32_t d1 = (uint32_t)hdr[1], d2 = (uint32_t)hdr[2], d3 = (uint32_t)hdr[3];
    const uint32_t sc = h ? ((d3 & 0x0F0F0F0Fu) | ((d1 >> 2) & 0x30303030u)) : (d1 & 0x3F3F3F3Fu);
    const uint32_t mn = h ? (((d3 >> 4) & 0x0F0F0F0Fu) | ((d2 >> 2) & 0x30303030u)) : (d2 & 0x3F3F3F3Fu);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        u.sc[jj] = (int)((sc >> (8 * jj)) & 0xff);
        u.mn[jj] = (int)((mn >> (8 * jj)) & 0xff);
    }
}
// The unit's integers against record rec: isc = sum_j sc_j * (q_w . q_x over sub-block j), imn =
// sum_j m_j * (sum of q_x over sub-block j), both over the whole super-block (the pair of lanes).
X100_DEV void q4k_half_sums(const Q4kHalf &u, const uint8_t *rec, int h, int &isc, int &imn)
{
    const v4i *xq = (const v4i *)(rec + 128 * h);
    int dj[4];
#pragma unroll
    for (int p = 0; p < 2; p++) {   // planes 2p, 2p+1: sub-blocks 4h + 2p (low), 4h + 2p + 1 (high)
        const v4i x0 = xq[4 * p], x1 = xq[4 * p + 1], x2 = xq[4 * p + 2], x3 = xq[4 * p + 3];
        int a = 0, b = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            a = dot4(u.lo[2 * p][t], x0[t], a);
            a = dot4(u.lo[2 * p + 1][t], x1[t], a);
            b = dot4(u.hi[2 * p][t], x2[t], b);
            b = dot4(u.hi[2 * p + 1][t], x3[t], b);
        }
        dj[2 * p] = a;
        dj[2 * p + 1] = b;
    }
    const v4i s32 = *(const v4i *)(rec + KR_S32 + 16 * h);
    isc = u.sc[0] * dj[0] + u.sc[1] * dj[1] + u.sc[2] * dj[2] + u.sc[3] * dj[3];
    imn = u.mn[0] * s32[0] + u.mn[1] * s32[1] + u.mn[2] * s32[2] + u.mn[3] * s32[3];
    isc += dpp_i<0xB1>(0, isc);   // + the other half
    imn += dpp_i<0xB1>(0, imn);
}
// The super-block's fp32 term (d, dmin of the weight block; dx of the record), in the oracle's
// operation order.
X100_DEV float q4k_term(float d, float dmin, float dx, int isc, int imn)
{
    const float dd = dx * d, dm = dx * dmin;
    return dd * (float)isc - dm * (float)imn;
}

// Blocks of kernel k that are resident on the whole device at once with lds bytes of dynamic LDS
// (the runtime's occupancy for the kernel times the CU count): the grid of a persistent launch.
// Cached per calling thread, keyed by (kernel address, block size, device, lds): template
// instances with the same signature are distinct kernels with distinct occupancy.
struct ResidentKey {
    const void *k;
    int nt, dev;
    size_t lds;
    int blocks;
};
template <typename Kern>
inline int resident_blocks(Kern k, int nt, size_t lds)
{
    static thread_local ResidentKey cache[16];
    static thread_local int used = 0, next = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const void *kp = (const void *)k;
    for (int i = 0; i < used; i++)
        if (cache[i].k == kp && cache[i].nt == nt && cache[i].dev == dev && cache[i].lds == lds)
            return cache[i].blocks;
    int occ = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, nt, lds) != hipSuccess || occ < 1) occ = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    ResidentKey &e = cache[used < 16 ? used++ : (next++ & 15)];
    e = ResidentKey{kp, nt, dev, lds, occ * cus};
    return e.blocks;
}
