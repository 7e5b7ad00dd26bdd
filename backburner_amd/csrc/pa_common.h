// pa_common.h - device helpers shared by the phone-attn HIP kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 pa_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 pa_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 pa_h8 __attribute__((ext_vector_type(8)));
typedef float pa_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t pa_u2 __attribute__((ext_vector_type(2)));
typedef uint32_t pa_u4 __attribute__((ext_vector_type(4)));

#define PA_LOG2E 1.4426950408889634f
#define PA_LN2 0.6931471805599453f

__device__ __forceinline__ pa_h2 pa_as_h2(uint32_t u) { return __builtin_bit_cast(pa_h2, u); }
__device__ __forceinline__ uint32_t pa_as_u32(pa_h2 h) { return __builtin_bit_cast(uint32_t, h); }

// v_perm_b32: byte k of the result = selector byte k; 0-3 pick bytes of `lo`, 4-7 bytes of `hi`, 12 = 0x00.
__device__ __forceinline__ uint32_t pa_perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// Four int8 (a dword of q8_0 quants) -> four integer-valued fp16 q (exact), in two packed halves (elements 0,1 and 2,3).
// Bias trick: q ^ 0x80 is q + 128 as an unsigned byte; 0x64XX as fp16 is 1024 + XX; minus 1152 gives q exactly.
__device__ __forceinline__ void pa_int_q8x4(uint32_t q, uint32_t & lo, uint32_t & hi) {
    const uint32_t x = q ^ 0x80808080u;
    const pa_h2 bias = {(_Float16) 1152.0f, (_Float16) 1152.0f};
    lo = pa_as_u32(pa_as_h2(pa_perm(0x64646464u, x, 0x04010400u)) - bias);
    hi = pa_as_u32(pa_as_h2(pa_perm(0x64646464u, x, 0x04030402u)) - bias);
}
// Four 4-bit values (masked to 0x0f0f0f0f) -> four integer-valued fp16 nib - 8 (exact).
__device__ __forceinline__ void pa_int_nib4(uint32_t n, uint32_t & lo, uint32_t & hi) {
    const pa_h2 bias = {(_Float16) 1032.0f, (_Float16) 1032.0f};
    lo = pa_as_u32(pa_as_h2(pa_perm(0x64646464u, n, 0x04010400u)) - bias);
    hi = pa_as_u32(pa_as_h2(pa_perm(0x64646464u, n, 0x04030402u)) - bias);
}
// Byte e of two dwords (two keys, same element) -> packed fp16 pair (key0, key1) of the biased value 1024 + byte.
__device__ __forceinline__ uint32_t pa_pair_byte(uint32_t x1, uint32_t x0, int e) {
    return pa_perm(x1, x0, 0x0c040c00u + (uint32_t) e * 0x00010001u) | 0x64006400u;
}

__device__ __forceinline__ float pa_f16_bits_to_f32(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }

// x as an opaque fp32 value in a register. A conversion to fp16 of a product would otherwise become v_fma_mix*_f16,
// which rounds the exact product to fp16 once; the reference rounds to fp32 first and then to fp16 (f2h(a * b)), and
// the two differ where the fp32 product sits on an fp16 rounding midpoint.
__device__ __forceinline__ float pa_f32(float x) { asm("" : "+v"(x)); return x; }

// Unaligned loads from a byte pointer (gfx9+ vector memory accepts byte-aligned dword addresses).
template <typename T> __device__ __forceinline__ T pa_ld(const uint8_t * p) { T v; __builtin_memcpy(&v, p, sizeof(T)); return v; }

__device__ __forceinline__ float pa_wave_max16x4(float v) {   // max over the 4 lanes {l, l^16, l^32, l^48}
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float pa_wave_sum16x4(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}
