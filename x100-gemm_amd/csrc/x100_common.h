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
enum { X100_Q4_0 = 2, X100_Q3_K = 11, X100_Q4_K = 12 };

// fp16 bits -> fp32 (exact).
X100_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32 in the default rounding mode).
X100_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

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

// Wave-wide (64 lanes) reductions.
X100_DEV int wave_sum_i(int v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
X100_DEV float wave_max_f(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Device-side Q8 activation formats (kept in LDS or a workspace; internal to the library).
//   Q8_0 (per 32): fp16 d, int8 q[32], int sum(q)     -- quantize_q8_0_native rounding
//   Q8_K (per 256): fp32 d, int8 q[256], int bsum[16] -- pack_A_q3k rounding
// Quantize one 32-element block held by one thread (values v[0..31]).
X100_DEV float q8_0_scale(float amax) { return amax / 127.0f; }
X100_DEV int clamp_i8(int q) { return q > 127 ? 127 : (q < -128 ? -128 : q); }
