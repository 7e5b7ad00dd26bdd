// pa_ingest.hip - KV ingest on the device: the q8_0 / q4_0 quantizers, and APPEND into HBM pages (gfx950).
//
//   quantize_kernel        ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref over contiguous 32-blocks
//   append_quant_kernel    fp32 K/V rows [n][nkv][hd] quantized (or converted to f16) straight into page rows: the
//                          sender's quantization of new keys, with no host round trip
//   append_f16_kernel      received q8_0 rows stored as f16 rows (the server's store_f16 mode, store_rows,
//                          phone-attn.h:305-319)
// The plain APPEND copy (phone-attn.h:403-421) is a device copy per page segment, issued by the host code.
//
// One thread per 32-value block; every float expression rounds as written (no contraction), as the oracle's C
// restatement does. The work is a byte stream: HBM-bound, a few µs for a 512-token APPEND.
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

// one 32-block of fp32 values -> its q8_0 (34 B) / q4_0 (18 B) / f16 (64 B) bytes
__device__ __forceinline__ void quant_block(int fmt, const float * xb, uint8_t * o) {
    #pragma clang fp contract(off)
    if (fmt == 1) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16) d);
        o[0] = (uint8_t) (dh & 0xff); o[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) (int8_t) roundf(xb[j] * id);
    } else if (fmt == 2) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++) { const float v = xb[j]; if (amax < fabsf(v)) { amax = fabsf(v); mx = v; } }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        // d = 0 / -8 is -0 (fp16 0x8000); keep the sign bit explicitly (a fused f32->f16 multiply-add would drop it)
        const uint16_t dh = d == 0.0f ? (uint16_t) ((__builtin_bit_cast(uint32_t, mx) >> 16) & 0x8000u) ^ 0x8000u
                                      : __builtin_bit_cast(uint16_t, (_Float16) d);
        o[0] = (uint8_t) (dh & 0xff); o[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < 16; j++) {
            const float x0 = xb[j] * id, x1 = xb[16 + j] * id;
            int q0 = (int8_t) (x0 + 8.5f), q1 = (int8_t) (x1 + 8.5f);
            q0 = q0 > 15 ? 15 : q0;
            q1 = q1 > 15 ? 15 : q1;
            o[2 + j] = (uint8_t) (q0 | (q1 << 4));
        }
    } else {
        for (int j = 0; j < 32; j++) {
            const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16) xb[j]);
            o[2 * j] = (uint8_t) (h & 0xff); o[2 * j + 1] = (uint8_t) (h >> 8);
        }
    }
}

__global__ __launch_bounds__(256) void quantize_kernel(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nblk, int fmt) {
    const int64_t b = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    quant_block(fmt, x + b * 32, y + b * (fmt == 1 ? 34 : 18));
}

// thread -> (tensor K/V, row j, head h, block b); rows j of the segment land at dst + j*rs
__global__ __launch_bounds__(256) void append_quant_kernel(const AppendArgs a) {
    const uint32_t nb = a.hd / 32, per_t = a.n * a.nkv * nb;
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    if (t >= 2 * per_t) return;
    const uint32_t tensor = t / per_t, u = t % per_t;
    const uint32_t j = u / (a.nkv * nb), h = (u / nb) % a.nkv, b = u % nb;
    const float * xb = (const float *) (tensor ? a.vsrc : a.ksrc) + ((size_t) j * a.nkv + h) * a.hd + 32 * b;
    const uint32_t bb = a.fmt == 1 ? 34 : a.fmt == 2 ? 18 : 64;
    uint8_t * o = (tensor ? a.vdst : a.kdst) + (size_t) j * a.rs + (size_t) h * a.hb + (size_t) b * bb;
    quant_block(a.fmt, xb, o);
}

// received q8_0 block -> 32 f16 values f16(d * q) (d * q is exact in fp32, so the one rounding is the reference's)
__global__ __launch_bounds__(256) void append_f16_kernel(const AppendArgs a) {
    const uint32_t nb = a.hd / 32, per_t = a.n * a.nkv * nb;
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    if (t >= 2 * per_t) return;
    const uint32_t tensor = t / per_t, u = t % per_t;
    const uint32_t j = u / (a.nkv * nb), h = (u / nb) % a.nkv, b = u % nb;
    const uint8_t * blk = (const uint8_t *) (tensor ? a.vsrc : a.ksrc) + (size_t) j * a.src_rs + (size_t) h * a.src_hb + 34 * b;
    const float d = pa_f16_bits_to_f32((uint16_t) (blk[0] | (blk[1] << 8)));
    uint8_t * o = (tensor ? a.vdst : a.kdst) + (size_t) j * a.rs + (size_t) h * a.hb + 64 * (size_t) b;
    for (int i = 0; i < 32; i++) {
        const uint16_t hv = __builtin_bit_cast(uint16_t, (_Float16) (d * (float) (int8_t) blk[2 + i]));
        o[2 * i] = (uint8_t) (hv & 0xff); o[2 * i + 1] = (uint8_t) (hv >> 8);
    }
}

hipError_t launch_quantize(int fmt, const float * x, void * y, int64_t n, hipStream_t st) {
    const int64_t nblk = n / 32;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_kernel, dim3((uint32_t) ((nblk + 255) / 256)), dim3(256), 0, st, x, (uint8_t *) y, nblk, fmt);
    return hipGetLastError();
}

hipError_t launch_append(bool from_f32, const AppendArgs & a, hipStream_t st) {
    const uint64_t threads = 2ull * a.n * a.nkv * (a.hd / 32);
    if (threads == 0) return hipSuccess;
    const dim3 grid((uint32_t) ((threads + 255) / 256));
    if (from_f32) hipLaunchKernelGGL(append_quant_kernel, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(append_f16_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace pa_hip
