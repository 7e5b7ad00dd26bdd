// pa_ingest.hip - KV ingest on the device: the q8_0 / q4_0 quantizers, and APPEND into HBM pages (gfx950).
//
//   quantize_kernel        ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref over contiguous 32-blocks
//   append_quant_kernel    fp32 K/V rows [n][nkv][hd] quantized (or converted to f16) straight into page rows: the
//                          sender's quantization of new keys, with no host round trip
//   append_f16_kernel      received q8_0 rows stored as f16 rows (the server's store_f16 mode, store_rows,
//                          phone-attn.h:305-319)
// The plain APPEND copy (phone-attn.h:403-421) is a device copy per page segment, issued by the host code.
//
// 16 lanes per 32-value block (details below). The work is a byte stream: HBM-bound, a few µs for a 512-token APPEND.
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

// One 32-block per 16 lanes (a row of the wave), lane l holding values 2l and 2l+1: coalesced loads, the block's
// amax by a 16-lane reduction, 16-bit (q8_0, q4_0) or 32-bit (f16) stores. Every float expression rounds as written
// (no contraction), as ggml's reference quantizers and the oracle's C restatement do.
template <int CTRL> __device__ __forceinline__ uint32_t ing_dpp(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, 0xf, 0xf, false);
}
// max over the 16 lanes of a row (quad swaps, then rotations by 4 and 8)
__device__ __forceinline__ float ing_rowmax16(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, ing_dpp<0xb1>(__builtin_bit_cast(uint32_t, v))));
    v = fmaxf(v, __builtin_bit_cast(float, ing_dpp<0x4e>(__builtin_bit_cast(uint32_t, v))));
    v = fmaxf(v, __builtin_bit_cast(float, ing_dpp<0x124>(__builtin_bit_cast(uint32_t, v))));
    v = fmaxf(v, __builtin_bit_cast(float, ing_dpp<0x128>(__builtin_bit_cast(uint32_t, v))));
    return v;
}
__device__ __forceinline__ unsigned long long ing_rowmax16_u64(unsigned long long v) {
    #pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const unsigned long long o = __shfl_xor(v, m);
        v = o > v ? o : v;
    }
    return v;
}

// block values x0 = xb[2l], x1 = xb[2l+1] (l = lane within the block's 16) -> the block's bytes at o
__device__ __forceinline__ void quant_block16(int fmt, float x0, float x1, int l, uint8_t * o) {
    #pragma clang fp contract(off)
    if (fmt == 1) {                                                  // quantize_row_q8_0_ref
        const float amax = ing_rowmax16(fmaxf(fabsf(x0), fabsf(x1)));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int q0 = (int) roundf(x0 * id), q1 = (int) roundf(x1 * id);
        *(uint16_t *) (o + 2 + 2 * l) = (uint16_t) (((uint32_t) q0 & 0xffu) | (((uint32_t) q1 & 0xffu) << 8));
        if (l == 0) *(uint16_t *) o = __builtin_bit_cast(uint16_t, (_Float16) d);
    } else if (fmt == 2) {                                           // quantize_row_q4_0_ref
        // the first value of the largest magnitude (a serial `if (amax < |v|)` scan from amax = 0, max = 0): 64-bit key
        // (|v| bits, 31 - index, sign), NaN never taken; no value above 0 leaves max = +0
        auto key = [](float v, uint32_t idx) -> unsigned long long {
            const uint32_t u = __builtin_bit_cast(uint32_t, v);
            const uint32_t a = v != v ? 0u : (u & 0x7fffffffu);
            return ((unsigned long long) a << 32) | ((unsigned long long) (31u - idx) << 1) | (u >> 31);
        };
        const unsigned long long k0 = key(x0, 2 * l), k1 = key(x1, 2 * l + 1);
        const unsigned long long k = ing_rowmax16_u64(k0 > k1 ? k0 : k1);
        const uint32_t ab = (uint32_t) (k >> 32);
        const float mx = ab == 0u ? 0.0f : __builtin_bit_cast(float, ab | ((uint32_t) (k & 1u) << 31));
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        // d = 0 / -8 is -0 (fp16 0x8000); keep the sign bit explicitly (a fused f32->f16 multiply-add would drop it)
        const uint16_t dh = d == 0.0f ? (uint16_t) ((__builtin_bit_cast(uint32_t, mx) >> 16) & 0x8000u) ^ 0x8000u
                                      : __builtin_bit_cast(uint16_t, (_Float16) d);
        int q0 = (int8_t) (x0 * id + 8.5f), q1 = (int8_t) (x1 * id + 8.5f);
        q0 = q0 > 15 ? 15 : q0;
        q1 = q1 > 15 ? 15 : q1;
        // byte j = q(j) | q(j + 16) << 4: lanes 0-7 take the quants of lane l + 8 (values 2l + 16, 2l + 17)
        const uint32_t qq = ((uint32_t) q0 & 0xffu) | (((uint32_t) q1 & 0xffu) << 8);
        const uint32_t hi = (uint32_t) __shfl_xor((int) qq, 8);
        if (l < 8) *(uint16_t *) (o + 2 + 2 * l) = (uint16_t) (qq | (hi << 4));
        if (l == 0) *(uint16_t *) o = dh;
    } else {
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16) x0), h1 = __builtin_bit_cast(uint16_t, (_Float16) x1);
        *(uint32_t *) (o + 4 * l) = h0 | (h1 << 16);
    }
}

// contiguous 32-blocks: block b of x -> y + b * (34 / 18) bytes
__global__ __launch_bounds__(256) void quantize_kernel(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nblk, int fmt) {
    const int64_t b = ((int64_t) blockIdx.x * 256 + threadIdx.x) / 16;
    const int l = threadIdx.x % 16;
    if (b >= nblk) return;                                           // whole 16-lane rows leave together
    const float * xb = x + b * 32;
    quant_block16(fmt, xb[2 * l], xb[2 * l + 1], l, y + b * (fmt == 1 ? 34 : 18));
}

// block u of the segment -> (tensor K/V, row j, head h, block b); rows j of the segment land at dst + j*rs
__global__ __launch_bounds__(256) void append_quant_kernel(const AppendArgs a) {
    const uint32_t nb = a.hd / 32, per_t = a.n * a.nkv * nb;
    const uint32_t t = (blockIdx.x * 256 + threadIdx.x) / 16;
    const int l = threadIdx.x % 16;
    if (t >= 2 * per_t) return;                                      // whole 16-lane rows leave together
    const uint32_t tensor = t / per_t, u = t % per_t;
    const uint32_t j = u / (a.nkv * nb), h = (u / nb) % a.nkv, b = u % nb;
    const float * xb = (const float *) (tensor ? a.vsrc : a.ksrc) + ((size_t) j * a.nkv + h) * a.hd + 32 * b;
    const uint32_t bb = a.fmt == 1 ? 34 : a.fmt == 2 ? 18 : 64;
    uint8_t * o = (tensor ? a.vdst : a.kdst) + (size_t) j * a.rs + (size_t) h * a.hb + (size_t) b * bb;
    quant_block16(a.fmt, xb[2 * l], xb[2 * l + 1], l, o);
}

// received q8_0 block -> 32 f16 values f16(d * q) (d * q is exact in fp32, so the one rounding is the reference's);
// lane l converts quants 2l, 2l+1
__global__ __launch_bounds__(256) void append_f16_kernel(const AppendArgs a) {
    const uint32_t nb = a.hd / 32, per_t = a.n * a.nkv * nb;
    const uint32_t t = (blockIdx.x * 256 + threadIdx.x) / 16;
    const int l = threadIdx.x % 16;
    if (t >= 2 * per_t) return;
    const uint32_t tensor = t / per_t, u = t % per_t;
    const uint32_t j = u / (a.nkv * nb), h = (u / nb) % a.nkv, b = u % nb;
    const uint8_t * blk = (const uint8_t *) (tensor ? a.vsrc : a.ksrc) + (size_t) j * a.src_rs + (size_t) h * a.src_hb + 34 * b;
    const float d = pa_f16_bits_to_f32((uint16_t) (blk[0] | (blk[1] << 8)));
    const float v0 = d * (float) (int8_t) blk[2 + 2 * l], v1 = d * (float) (int8_t) blk[3 + 2 * l];
    uint8_t * o = (tensor ? a.vdst : a.kdst) + (size_t) j * a.rs + (size_t) h * a.hb + 64 * (size_t) b;
    const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16) v0), h1 = __builtin_bit_cast(uint16_t, (_Float16) v1);
    *(uint32_t *) (o + 4 * l) = h0 | (h1 << 16);
}

hipError_t launch_quantize(int fmt, const float * x, void * y, int64_t n, hipStream_t st) {
    const int64_t nblk = n / 32;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_kernel, dim3((uint32_t) ((nblk * 16 + 255) / 256)), dim3(256), 0, st, x, (uint8_t *) y, nblk, fmt);
    return hipGetLastError();
}

hipError_t launch_append(bool from_f32, const AppendArgs & a, hipStream_t st) {
    const uint64_t threads = 16ull * 2 * a.n * a.nkv * (a.hd / 32);    // 16 lanes per 32-block
    if (threads == 0) return hipSuccess;
    const dim3 grid((uint32_t) ((threads + 255) / 256));
    if (from_f32) hipLaunchKernelGGL(append_quant_kernel, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(append_f16_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace pa_hip
