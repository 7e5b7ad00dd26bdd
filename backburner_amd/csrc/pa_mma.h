// pa_mma.h - device helpers shared by the matrix-core attention kernels (pa_mma.hip: head dim 128;
// pa_mma256.hip: head dim 256): raw K/V staging units and their fp16 dequantization, the LDS-only barrier, lane
// reductions and the scalar page cursor.
#pragma once
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

typedef _Float16 mm_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mm_h2 __attribute__((ext_vector_type(2)));
typedef float mm_f16 __attribute__((ext_vector_type(16)));
typedef int mm_i4 __attribute__((ext_vector_type(4)));
typedef int mm_i16 __attribute__((ext_vector_type(16)));
typedef __fp16 mm_tr4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
#define MM_LDS __attribute__((address_space(3)))

constexpr float MM_PMAX = 6.0f;                   // p <= 2^6 between rescales
constexpr float MM_LOG2E = 1.4426950408889634f;

template <int FMT> struct MmFmt {
    static constexpr int BB = FMT == 1 ? 34 : FMT == 2 ? 18 : 64;    // bytes per 32-value block
};

// raw bytes of one staging unit = (tensor, key, block, half): 16 values of one 32-block and the block scale
template <int FMT> struct MmRaw {
    pa_u4 q[FMT == 0 ? 2 : 1];
    uint32_t d;
};

// One unit through a buffer resource (the tile's scalar base, its valid bytes as the range) and a 32-bit offset
template <int FMT>
__device__ __forceinline__ void mm_load_unit_buf(MmRaw<FMT> & r, __amdgpu_buffer_rsrc_t rsrc, uint32_t off, int half) {
    if constexpr (FMT == 1) {
        r.q[0] = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 2 + 16 * half, 0, 0));
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
    } else if constexpr (FMT == 2) {
        r.q[0] = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 2, 0, 0));
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
    } else {
        r.q[0] = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 32 * half, 0, 0));
        r.q[1] = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 32 * half + 16, 0, 0));
        r.d = 0;
    }
}

// The same unit with the quantized formats' 16 value bytes read at an even-aligned address: a 16-byte load at
// addr & ~2 and a 2-byte load of the unit's last two bytes, joined by byte alignment (q8_0 / q4_0 blocks are 34 / 18
// bytes, so every other block's values start 2 bytes past a dword boundary, and a 16-byte load there takes the
// memory pipeline's slow unaligned path). No byte outside the unit is read. base_lo = the low bits of the buffer's
// base address; any alignment gives the right bytes (an odd one through the slow path).
template <int FMT>
__device__ __forceinline__ void mm_load_unit_buf_al(MmRaw<FMT> & r, __amdgpu_buffer_rsrc_t rsrc, uint32_t off, int half,
                                                    uint32_t base_lo) {
    if constexpr (FMT == 0) {
        mm_load_unit_buf<FMT>(r, rsrc, off, half);
    } else {
        const uint32_t q = off + 2 + (FMT == 1 ? 16 * half : 0);         // the 16 value bytes
        const uint32_t sh = (base_lo + q) & 2u;
        const pa_u4 w = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, q - sh, 0, 0));
        const uint32_t t = __builtin_amdgcn_raw_buffer_load_b16(rsrc, q + 14, 0, 0);
        r.q[0] = (pa_u4){__builtin_amdgcn_alignbyte(w[1], w[0], sh), __builtin_amdgcn_alignbyte(w[2], w[1], sh),
                         __builtin_amdgcn_alignbyte(w[3], w[2], sh), __builtin_amdgcn_alignbyte(t, w[3], sh)};
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
    }
}

// 16 values -> fp16 (8 dwords). Quantized formats: byte u (unsigned quant) -> fp16 bits 0x6400 | u = 1024 + u exactly,
// minus (1024 + bias) exactly, times d (one rounding); with INT the integer quants themselves (exact, no rounding).
template <int FMT, bool INT = false>
__device__ __forceinline__ void mm_dequant(const MmRaw<FMT> & r, int half, pa_u4 & lo, pa_u4 & hi) {
    if constexpr (FMT == 0) {
        lo = r.q[0]; hi = r.q[1];
    } else {
        pa_u4 u = r.q[0];
        if constexpr (FMT == 1) {
            u = u ^ 0x80808080u;                                          // int8 -> uint8 (q + 128)
        } else {
            const int sh = 4 * half;                                      // q4_0: low nibbles = values 0-15
            u = (u >> sh) & 0x0f0f0f0fu;
        }
        constexpr float bias = FMT == 1 ? 1152.0f : 1032.0f;              // 1024 + 128 / 1024 + 8
        const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t) r.d);
        const mm_h2 d2 = {dh, dh}, b2 = {(_Float16) bias, (_Float16) bias};
        uint32_t w[8];
        #pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t x = u[c];
            const mm_h2 a = __builtin_bit_cast(mm_h2, pa_perm(0x64646464u, x, 0x04010400u));   // bytes 0, 1
            const mm_h2 b = __builtin_bit_cast(mm_h2, pa_perm(0x64646464u, x, 0x04030402u));   // bytes 2, 3
            if constexpr (INT) {
                w[2 * c] = __builtin_bit_cast(uint32_t, (mm_h2) (a - b2));
                w[2 * c + 1] = __builtin_bit_cast(uint32_t, (mm_h2) (b - b2));
            } else {
                w[2 * c] = __builtin_bit_cast(uint32_t, (mm_h2) ((a - b2) * d2));
                w[2 * c + 1] = __builtin_bit_cast(uint32_t, (mm_h2) ((b - b2) * d2));
            }
        }
        lo = (pa_u4){w[0], w[1], w[2], w[3]};
        hi = (pa_u4){w[4], w[5], w[6], w[7]};
    }
}

__device__ __forceinline__ void mm_lds_barrier() {   // LDS-only workgroup barrier: loads in flight are not waited for
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// v_permlane32_swap of a value with itself gives every lane the pair (value of lane l % 32, value of lane l % 32 + 32)
__device__ __forceinline__ float mm_max32(float v) {    // max over lanes l and l ^ 32
    const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned) t[0]), __builtin_bit_cast(float, (unsigned) t[1]));
}
__device__ __forceinline__ float mm_sum32(float v) {    // sum over lanes l and l ^ 32
    const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return __builtin_bit_cast(float, (unsigned) t[0]) + __builtin_bit_cast(float, (unsigned) t[1]);
}

// Page cursor (scalar): the page holding a tile, its tile range and key count. A cursor moves only when a tile leaves
// its page, so the common case reads no kernel argument memory (whose scalar loads would also wait for the LDS
// operations in flight).
struct MmCursor {
    uint32_t pg, tb, te, nk;
    const uint8_t * kb, * vb;
    __device__ __forceinline__ void init(const AttnArgs & a) {
        pg = 0; tb = a.cstart[0]; te = a.cstart[1]; nk = a.pstart[1] - a.pstart[0]; kb = a.kp[0]; vb = a.vp[0];
    }
    __device__ __forceinline__ void seek(const AttnArgs & a, uint32_t tau) {
        while (tau >= te) {
            pg++;
            tb = te;
            te = a.cstart[pg + 1];
            nk = a.pstart[pg + 1] - a.pstart[pg];
            kb = a.kp[pg];
            vb = a.vp[pg];
            __builtin_amdgcn_s_waitcnt(0xc07f);                      // lgkmcnt(0): no scalar load left outstanding
        }
    }
};

}  // namespace pa_hip
