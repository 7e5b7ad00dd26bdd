// pa_attn.h - kernel argument blocks and launchers of the phone-attn HIP kernels (internal to libpa_hip.so).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/phone_attn_hip.h"

namespace pa_hip {

constexpr int MAXP = 128;  // pages per attention launch (more are split over several launches into one slot array): 512k
                           // keys in 4,096-key pages, with the kernel arguments under 4 KB

struct AttnArgs {
    const uint8_t * kp[MAXP];       // page base (key 0, head 0) of K / V
    const uint8_t * vp[MAXP];
    uint32_t pstart[MAXP + 1];      // key prefix: page p holds keys [pstart[p], pstart[p+1]) of the call
    uint32_t cstart[MAXP + 1];      // decode kernel: 32-key tile prefix, page p holds tiles [cstart[p], cstart[p+1])
    uint32_t ptl;                   // log2 of the tiles per page when every page but the last holds that same power of
                                    // two of 32-key tiles (the last one any number), else 32: pages by shift, no table walk
    uint32_t n_pages, n_chunks, chunk, n_items;   // chunk = keys per workgroup; n_items = chunks x heads x row blocks
                                                  // (decode kernel: n_chunks = tile groups, chunk = 32, items = groups x pairs)
    uint32_t rs, hb, nkv;
    uint32_t rows;                  // real query rows per KV head
    uint32_t qr;                    // padded rows per KV head in the slots
    uint32_t nrb;                   // row blocks per KV head
    uint32_t slot0;                 // slot of chunk 0 of this launch
    uint32_t slots;                 // decode / MMA kernels: the call's slot count (slots are row-major: [head, row][slot])
    uint32_t qmode;                 // PA_QMODE_GGML / PA_QMODE_F16
    uint32_t fused;                 // 1: this launch holds every chunk of the call (a single chunk writes the result)
    float scale;                    // softmax scale (PA_QMODE_F16 folds it into Q)
    float s_mul;                    // factor from the dot to base-2 logits (scale * log2 e, or log2 e)
    const float * q;                // [nkv][rows][hd] fp32
    float * po;                     // slots [nkv][qr][slots][hd]
    float2 * pml;                   // the same without hd: (max in base-2 units, sum)
    float * O, * m, * l;            // final [nkv][rows][hd], [nkv][rows]
};
static_assert(sizeof(AttnArgs) <= 4096, "the page table travels in the kernel arguments");

struct MergeArgs {
    const float * po;
    const float2 * pml;
    float * O, * m, * l;            // [nkv][rows][hd], [nkv][rows]
    uint32_t n_slots, nkv, qr, rows;
    uint64_t sst = 0, rst = 0;      // slot s of output row h*qr + i at s*sst + (h*qr + i)*rst (rows of hd floats / one float2)
    uint16_t * Oh = nullptr;        // non-null: write the reply format instead of (O, m, l): Oh = f16(O / l) [nkv][rows][hd]
    float * lse = nullptr;          // and lse = m + log l [nkv][rows] (0 and -inf where l = 0)
};

hipError_t launch_merge(int hd, const MergeArgs & a, hipStream_t st);
hipError_t launch_decode(int fmt, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0 = nullptr,
                         hipEvent_t ev1 = nullptr);
hipError_t launch_mma(int fmt, int nw, bool skip, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0 = nullptr,
                      hipEvent_t ev1 = nullptr);
hipError_t launch_mma256(int fmt, bool skip, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0 = nullptr,
                         hipEvent_t ev1 = nullptr);
hipError_t launch_quantize(int fmt, const float * x, void * y, int64_t n, hipStream_t st);

struct AppendArgs {                 // one page segment of an APPEND: rows j = 0 .. n-1
    uint8_t * kdst, * vdst;         // the segment's first row in the K / V page
    const void * ksrc, * vsrc;      // fp32 [n][nkv][hd] (append_quant_kernel) or received rows (append_f16_kernel)
    uint32_t n, nkv, hd;
    uint32_t rs, hb;                // stored row and head strides (bytes)
    uint32_t src_rs, src_hb;        // received row and head strides (append_f16_kernel)
    int fmt;                        // stored format (append_quant_kernel)
};
hipError_t launch_append(bool from_f32, const AppendArgs & a, hipStream_t st);
hipError_t launch_merge_partial(int hd, float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                                uint64_t rows, hipStream_t st);
hipError_t launch_normalise(int hd, const float * O, const float * m, const float * l, uint64_t rows, uint16_t * Oh,
                            float * lse, hipStream_t st);
hipError_t launch_coattn(int hd, const uint16_t * Oh, const float * lse, const float * Oloc, const float * mloc,
                         const float * lloc, uint64_t rows, float * out, float * lse_out, hipStream_t st);

#ifndef PA_ACCEPT_SEG
#define PA_ACCEPT_SEG 16384
#endif
// logits per acceptance workgroup (a multiple of 1024). [17][151936] fp32: 7.2 us at 16384 (170 workgroups), 8.3 at
// 8192, 8.8 at 32768, 12.0 at 4096 - fewer, fuller workgroups, and fewer keys for the last one to fold
constexpr int ACCEPT_SEG = PA_ACCEPT_SEG;

struct AcceptArgs {
    const float * logits;
    const int32_t * draft;
    int32_t * out;                  // [2 + n_rows]
    unsigned long long * part;      // [n_rows][splits] packed (orderable value, ~index)
    unsigned int * counter;         // one counter, zero between calls (the last block resets it)
    int64_t vocab;
    int n_rows, splits;
};
hipError_t launch_accept(const AcceptArgs & a, hipStream_t st);

// host side (pa_abi.cpp): the calling thread's last error, and the engine-path call with its split-K slots in a fixed
// device array of `cap` bytes instead of a workspace (nothing allocated; the split adapts so the slots fit, and a call
// whose launches cannot fit one slot set each is refused)
void set_error(const std::string & e);
int attn_fixed_scratch(char * scratch, size_t cap, const pa_hip_shape * s, const void * const * k_pages,
                       const void * const * v_pages, const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m,
                       float * l, hipStream_t st);

}  // namespace pa_hip
